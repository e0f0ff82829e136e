"""CPU oracle for the MXFP4 expert / latent-MLA / KDA decode path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path (the ``k3hip`` package and
``libk3hip.so``) imports, links or calls this package.  Its only legitimate users are
``tests/``, ``__graft_entry__.smoke()`` (to check the HIP result) and the
``cpu_baseline`` leg of ``bench.py`` (a timed CPU restatement of the reference CPU path).

Modules
-------
``mxfp4``        E2M1/E8M0 decode (bit-exact restatement of ``k3ref/weights.py:29-37``),
                 fp64 matvec oracle, the reference's unfused dequant-then-matmul definition
                 (``air_llm/models/kimi_k3/mxfp4.py:84-92``), and a bf16 RNE helper.
``moe``          routers (softmax top-k; sigmoid + correction bias per
                 ``k3ref/layers.py:214-224``), SwiGLU/SiTU expert FFN
                 (``k3ref/layers.py:226-239``), routed + shared layer combine
                 (``k3ref/layers.py:241-261`` without the K3 latent wrapper).
``mla``          absorbed latent-MLA decode core (``attention_mla.py:193-212``) and the
                 expanded form it must equal (``k3ref/layers.py:152-185``), both fp64.
``kda``          Kimi Delta Attention: the recurrence (``attention_kda.py:65-90``), the short
                 convolution, L2 and gated RMS norms (``ops.py:31-60``) and the whole layer
                 (``attention_kda.py:94-115``), fp64.
``cpu_baseline`` torch-CPU fp32 restatement of the k3ref path, timed by ``bench.py``.
``native``       ctypes loader for ``mxfp4_ref.c``: an independent C restatement of the
                 decode and of the reference Metal kernel's sequential fp32 FMA order
                 (``air_llm/kernels/metal/mxfp4_matvec.py:29-63``).

Pinning (how each function is checked independently of its own formula) is described
in each module's docstring and exercised by ``tests/test_oracle_*.py``.
"""
