"""Checkpoint ingestion into the resident expert table -- the counterpart of the
reference's ``TensorSource`` (air_llm/models/kimi_k3/loader.py:47-266) and of the
records its manifest builder writes (tools/k3_manifest.py:87-143), for the tensors the
MoE decode path reads.

* A safetensors shard is parsed from its header only: an 8-byte little-endian header
  length, a JSON header, then the data region the header's ``data_offsets`` index.  A
  header length larger than the file or than 256 MiB is rejected (k3_manifest.py:87-92).
* Tensor records carry the fields of the reference manifest (name, file, offset, nbytes,
  shape, dtype), so ``TensorSource(manifest=...)`` accepts a reference
  ``manifest.jsonl.gz`` as is, and ``TensorSource(ckpt=...)`` scans the shards' headers
  itself.
* ``expert_source(layer, expert, which)`` returns one MXFP4 projection ``(packed, scales)``
  as device tensors.  When ``weight_scale`` starts where ``weight_packed`` ends (every
  shard the reference checked, loader.py:232-236) the pair is one contiguous read, else
  two (loader.py:243-266); the scale guard of ``assert_scales_representable`` runs on
  every fetched projection (loader.py:246-247).
* Reads land in page-locked host buffers and reach the GPU by asynchronous copies on a
  copy stream of default priority, with two staging buffers in flight, so the file read
  of one projection overlaps the host-to-device copy of the previous one (four reader
  threads with their own buffers in ``load_experts``).
  ``load_experts(layer, n)`` makes a layer's experts resident in one device allocation
  (each projection keeps the file's [packed | scales] order) and checks every scale
  region on the device with one host synchronisation per layer.

SSD streaming policy (which experts to keep, prefetch, eviction) is the caller's; this
module moves bytes and keeps the counters the reference keeps (``bytes_read``,
``expert_bytes``, ``experts_loaded``).
"""
from __future__ import annotations

import gzip
import json
import struct
from pathlib import Path

import numpy as np
import torch

from . import _lib
from . import _torch as T

MAX_HEADER = 256 * 2 ** 20
DTYPES = {"F32": (np.float32, torch.float32), "BF16": (np.uint16, torch.bfloat16),
          "F16": (np.float16, torch.float16), "U8": (np.uint8, torch.uint8),
          "I8": (np.int8, torch.int8), "I32": (np.int32, torch.int32), "I64": (np.int64, torch.int64)}
MOE_KEYS = ("gate.weight", "gate.e_score_correction_bias",
            "routed_expert_down_proj.weight", "routed_expert_up_proj.weight",
            "routed_expert_norm.weight", "shared_experts.gate_proj.weight",
            "shared_experts.up_proj.weight", "shared_experts.down_proj.weight")   # loader.py:30-33
WHICH = ("w1", "w3", "w2")        # gate, up, down (loader.py:229; moe.py:79-88)
_ALIGN = 256


def expert_name(layer: int, expert: int, which: str) -> str:
    """Tensor-name stem of one routed projection (loader.py:238-239)."""
    return f"language_model.model.layers.{layer}.block_sparse_moe.experts.{expert}.{which}"


def moe_prefix(layer: int) -> str:
    return f"language_model.model.layers.{layer}.block_sparse_moe."


def read_header(path) -> tuple[dict, int]:
    """(header, data_base) of a safetensors file; data_base is the file offset of the data
    region (8 + header length)."""
    path = Path(path)
    size = path.stat().st_size
    with path.open("rb") as fh:
        raw = fh.read(8)
        if len(raw) != 8:
            raise ValueError(f"Invalid safetensors file (no header length): {path.name}")
        n = struct.unpack("<Q", raw)[0]
        if n > size - 8 or n > MAX_HEADER:
            raise ValueError(f"Invalid safetensors header size: {path.name}")
        return json.loads(fh.read(n)), 8 + n


def scan_checkpoint(ckpt, pattern: str = "*.safetensors") -> dict[str, dict]:
    """Manifest records for every tensor of every shard under ckpt (headers only)."""
    recs = {}
    for shard in sorted(Path(ckpt).glob(pattern)):
        hdr, base = read_header(shard)
        for name, t in hdr.items():
            if name == "__metadata__":
                continue
            s, e = t["data_offsets"]
            recs[name] = {"name": name, "file": shard.name, "offset": base + s, "nbytes": e - s,
                          "shape": list(t["shape"]), "dtype": t["dtype"]}
    return recs


def load_manifest(path) -> tuple[dict, dict[str, dict]]:
    """(meta, records by name) from a reference manifest.jsonl.gz (k3_manifest.py:99-143)."""
    meta, recs = {}, {}
    with gzip.open(path, "rt") as fh:
        for line in fh:
            r = json.loads(line)
            if r.get("__meta__"):
                meta = r
            else:
                recs[r["name"]] = r
    return meta, recs


def write_safetensors(path, tensors) -> None:
    """Write ``{name: (array, dtype)}`` as one safetensors file, data in the given order
    (so a projection's packed and scale tensors are adjacent when given one after the
    other).  bf16 arrays are passed as their uint16 bit patterns."""
    header, blobs, off = {}, [], 0
    for name, (arr, dtype) in tensors.items():
        a = np.ascontiguousarray(arr)
        if a.dtype != np.dtype(DTYPES[dtype][0]):
            raise TypeError(f"{name}: array dtype {a.dtype} does not store {dtype}")
        b = a.tobytes()
        header[name] = {"dtype": dtype, "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    hb = json.dumps(header, separators=(",", ":")).encode()
    hb += b" " * (-len(hb) % 8)
    with Path(path).open("wb") as fh:
        fh.write(struct.pack("<Q", len(hb)))
        fh.write(hb)
        for b in blobs:
            fh.write(b)


class _NotAdjacent(Exception):
    pass


class TensorSource:
    """Tensor access for the MoE decode path (loader.py:47-266).

    ``TensorSource(manifest=path)`` reads a reference manifest; ``TensorSource(ckpt=dir)``
    scans the shards under dir.  ``ckpt`` overrides the manifest's checkpoint directory.
    Host reads only (``host``, ``expert_host``) work without a GPU; ``tensor``,
    ``expert_source``, ``moe_weights`` and ``load_experts`` return device tensors."""

    def __init__(self, manifest=None, ckpt=None, device=None, stage_bytes: int = 32 << 20):
        if manifest is not None:
            self.meta, self.recs = load_manifest(manifest)
            root = ckpt or self.meta.get("checkpoint")
            if root is None:
                raise ValueError("the manifest names no checkpoint directory; pass ckpt=")
            self.ckpt = Path(root)
        elif ckpt is not None:
            self.meta, self.ckpt = {}, Path(ckpt)
            self.recs = scan_checkpoint(self.ckpt)
        else:
            raise ValueError("TensorSource needs manifest= or ckpt=")
        self.device = torch.device(device) if device is not None else None
        self.bytes_read = 0
        self.expert_bytes = 0
        self.experts_loaded = 0
        self.reads = 0
        self._files = {}
        self._stage_bytes = int(stage_bytes)
        self._stage = None           # two page-locked buffers, created on first device use
        self._stage_ev = [None, None]
        self._next = 0
        self._copy = None

    # ------------------------------------------------------------------ host reads
    def close(self) -> None:
        for fh in self._files.values():
            fh.close()
        self._files.clear()

    def _fh(self, file: str):
        fh = self._files.get(file)
        if fh is None:
            fh = self._files[file] = (self.ckpt / file).open("rb")
        return fh

    def record(self, name: str) -> dict:
        r = self.recs.get(name)
        if r is None:
            raise KeyError(f"tensor not in checkpoint: {name}")
        return r

    def _read_into(self, file: str, offset: int, out: np.ndarray) -> None:
        fh = self._fh(file)
        fh.seek(offset)
        n = fh.readinto(memoryview(out).cast("B"))
        if n != out.nbytes:
            raise ValueError(f"short read from {file} at {offset}: {n} of {out.nbytes} bytes")
        self.bytes_read += n
        self.reads += 1

    def host(self, name: str) -> np.ndarray:
        """One tensor as a host array of its stored dtype (bf16 as uint16 bit patterns)."""
        r = self.record(name)
        a = np.empty(r["shape"], dtype=DTYPES[r["dtype"]][0])
        self._read_into(r["file"], r["offset"], a)
        return a

    def _pair(self, base: str):
        ra = self.record(base + ".weight_packed")
        rb = self.record(base + ".weight_scale")
        if ra["dtype"] != "U8" or rb["dtype"] != "U8":
            raise ValueError(f"{base}: packed and scales must be U8")
        return ra, rb, ra["file"] == rb["file"] and ra["offset"] + ra["nbytes"] == rb["offset"]

    def expert_host(self, layer: int, expert: int, which: str):
        """(packed, scales) host arrays of one projection: one read when adjacent."""
        ra, rb, adjacent = self._pair(expert_name(layer, expert, which))
        before = self.bytes_read
        buf = np.empty(ra["nbytes"] + rb["nbytes"], dtype=np.uint8)
        if adjacent:
            self._read_into(ra["file"], ra["offset"], buf)
        else:
            self._read_into(ra["file"], ra["offset"], buf[:ra["nbytes"]])
            self._read_into(rb["file"], rb["offset"], buf[ra["nbytes"]:])
        self.experts_loaded += 1
        self.expert_bytes += self.bytes_read - before
        return (buf[:ra["nbytes"]].reshape(ra["shape"]), buf[ra["nbytes"]:].reshape(rb["shape"]))

    # ------------------------------------------------------------------ device side
    def _dev(self) -> torch.device:
        if self.device is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        return self.device

    def _staging(self, nbytes: int):
        """The next page-locked staging buffer, once the copy that last read it is done."""
        if self._copy is None:
            self._copy = torch.cuda.Stream(self._dev())
        if self._stage is None:
            self._stage = [None, None]
        i = self._next
        self._next ^= 1
        if self._stage_ev[i] is not None:
            self._stage_ev[i].synchronize()
            self._stage_ev[i] = None
        if self._stage[i] is None or self._stage[i].numel() < nbytes:
            self._stage[i] = torch.empty(max(nbytes, self._stage_bytes), dtype=torch.uint8, pin_memory=True)
        return i, self._stage[i]

    def _upload(self, i: int, host: torch.Tensor, dst: torch.Tensor) -> None:
        """Asynchronous host-to-device copy of a staging buffer on the copy stream."""
        self._copy.wait_stream(torch.cuda.current_stream(self._dev()))
        with torch.cuda.stream(self._copy):
            dst.copy_(host, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(self._copy)
        self._stage_ev[i] = ev
        dst.record_stream(self._copy)

    def _ready(self) -> None:
        """Make the caller's current stream wait for every upload issued so far."""
        if self._copy is not None:
            torch.cuda.current_stream(self._dev()).wait_stream(self._copy)

    def _fetch_pair(self, base: str, dst: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Read one projection into a staging buffer and upload it to dst ([packed|scales]
        bytes); returns the (packed, scales) device views."""
        ra, rb, adjacent = self._pair(base)
        na, nb = ra["nbytes"], rb["nbytes"]
        i, stage = self._staging(na + nb)
        host = stage[:na + nb]
        hv = host.numpy()
        if adjacent:
            self._read_into(ra["file"], ra["offset"], hv)
        else:
            self._read_into(ra["file"], ra["offset"], hv[:na])
            self._read_into(rb["file"], rb["offset"], hv[na:])
        self._upload(i, host, dst[:na + nb])
        return dst[:na].view(ra["shape"]), dst[na:na + nb].view(rb["shape"])

    def tensor(self, name: str, dtype: torch.dtype | None = None) -> torch.Tensor:
        """One tensor on the device (bf16 stays bf16), optionally cast."""
        r = self.record(name)
        i, stage = self._staging(r["nbytes"])
        host = stage[:r["nbytes"]]
        self._read_into(r["file"], r["offset"], host.numpy())
        raw = torch.empty(r["nbytes"], dtype=torch.uint8, device=self._dev())
        self._upload(i, host, raw)
        self._ready()
        t = raw.view(DTYPES[r["dtype"]][1]).view(r["shape"])
        return t if dtype is None else t.to(dtype)

    def moe_weights(self, layer: int) -> dict:
        """The non-expert MoE weights of a layer as device tensors (loader.py:284-285)."""
        p = moe_prefix(layer)
        return {k: self.tensor(p + k) for k in MOE_KEYS if (p + k) in self.recs}

    def expert_source(self, layer: int, expert: int, which: str):
        """One MXFP4 projection (packed [N, K/2], scales [N, K/32]) on the device, scale
        range checked (loader.py:229-249)."""
        ra, rb, _ = self._pair(expert_name(layer, expert, which))
        before = self.bytes_read
        dst = torch.empty(ra["nbytes"] + rb["nbytes"], dtype=torch.uint8, device=self._dev())
        packed, scales = self._fetch_pair(expert_name(layer, expert, which), dst)
        self._ready()
        self.experts_loaded += 1
        self.expert_bytes += self.bytes_read - before
        from .mxfp4 import assert_scales_representable
        assert_scales_representable(scales)
        return packed, scales

    def load_experts(self, layer: int, n_experts: int, whiches=WHICH) -> "ResidentExperts":
        """Every expert of a layer resident in one device allocation; the scale guard runs on
        the device for every projection and is checked with one synchronisation."""
        names = [(e, w) for e in range(n_experts) for w in whiches]
        sizes, offs, off = [], [], 0
        for e, w in names:
            ra, rb, _ = self._pair(expert_name(layer, e, w))
            n = ra["nbytes"] + rb["nbytes"]
            offs.append(off)
            sizes.append(n)
            off += -(-n // _ALIGN) * _ALIGN
        buf = torch.empty(off, dtype=torch.uint8, device=self._dev())
        mm = torch.empty((len(names), 2), dtype=torch.int32, device=self._dev())
        views = {}
        before = self.bytes_read
        self._load_parallel(layer, names, buf, offs, sizes, views)
        self._ready()
        st = torch.cuda.current_stream(self._dev())
        for j, (e, w) in enumerate(names):
            s = views[(e, w)][1]
            _lib.call("k3_scale_minmax", T.ptr(s), s.numel(), T.ptr(mm[j]), st.cuda_stream)
        lo_hi = mm.cpu().numpy()
        bad = np.nonzero((lo_hi[:, 0] < 2) | (lo_hi[:, 1] > 252))[0]
        if bad.size:
            e, w = names[int(bad[0])]
            lo, hi = lo_hi[bad[0]]
            raise ValueError(f"Unsupported MXFP4 scale range {lo}..{hi} in {expert_name(layer, e, w)}; "
                             "require 2..252 to avoid subnormal scales, overflow, and E8M0 NaN")
        self.experts_loaded += len(names)
        self.expert_bytes += self.bytes_read - before
        return ResidentExperts(layer, n_experts, buf, views)


    READERS = 4   # reader threads (and page-locked staging buffers) of load_experts

    def _load_parallel(self, layer, names, buf, offs, sizes, views) -> None:
        """Read the projections with READERS threads (positional reads on per-file
        descriptors, no shared file offset), each into its own page-locked buffer; the
        calling thread uploads them in order on the copy stream.  A buffer is refilled only
        after the copy that read it has finished."""
        import os
        from concurrent.futures import ThreadPoolExecutor
        if self._copy is None:
            self._copy = torch.cuda.Stream(self._dev())
        buf.record_stream(self._copy)  # written on the copy stream: not reused before those copies end
        nr = self.READERS
        cap = max(sizes)
        stages = [torch.empty(cap, dtype=torch.uint8, pin_memory=True) for _ in range(nr)]
        events = [None] * nr
        fds = {}

        def fd(file):
            f = fds.get(file)
            if f is None:
                f = fds[file] = os.open(self.ckpt / file, os.O_RDONLY)
            return f

        for e, w in names:                       # open every file on this thread first
            ra, rb, _ = self._pair(expert_name(layer, e, w))
            fd(ra["file"]), fd(rb["file"])

        def read(j):
            e, w = names[j]
            ra, rb, adjacent = self._pair(expert_name(layer, e, w))
            i = j % nr
            if events[i] is not None:
                events[i].synchronize()
            hv = memoryview(stages[i].numpy()).cast("B")
            na, nb = ra["nbytes"], rb["nbytes"]
            parts = [(ra, 0, na + nb)] if adjacent else [(ra, 0, na), (rb, na, nb)]
            for r, at, n in parts:
                got = os.preadv(fds[r["file"]], [hv[at:at + n]], r["offset"])
                if got != n:
                    raise ValueError(f"short read from {r['file']} at {r['offset']}: {got} of {n} bytes")
            return len(parts), na + nb

        try:
            with ThreadPoolExecutor(nr) as pool:
                fut = {j: pool.submit(read, j) for j in range(min(nr, len(names)))}
                for j, (e, w) in enumerate(names):
                    nreads, n = fut.pop(j).result()
                    self.reads += nreads
                    self.bytes_read += n
                    i = j % nr
                    ra, rb, _ = self._pair(expert_name(layer, e, w))
                    dst = buf[offs[j]:offs[j] + sizes[j]]
                    self._copy.wait_stream(torch.cuda.current_stream(self._dev()))
                    with torch.cuda.stream(self._copy):
                        dst.copy_(stages[i][:n], non_blocking=True)
                        ev = torch.cuda.Event()
                        ev.record(self._copy)
                    events[i] = ev
                    views[(e, w)] = (dst[:ra["nbytes"]].view(ra["shape"]),
                                     dst[ra["nbytes"]:ra["nbytes"] + rb["nbytes"]].view(rb["shape"]))
                    if j + nr < len(names):
                        fut[j + nr] = pool.submit(read, j + nr)
        finally:
            # every issued copy has finished before the staging buffers are reused or the
            # error propagates (buf is also marked as used on the copy stream)
            for ev in events:
                if ev is not None:
                    ev.synchronize()
            for f in fds.values():
                os.close(f)


class ResidentExperts:
    """A layer's experts resident in HBM: ``source`` has the ``expert_source`` signature
    (layer, expert, which) and returns device views, so ``RoutedMoE`` / ``LatentMoE`` build
    their pointer table from it without copies."""

    def __init__(self, layer: int, n_experts: int, buf: torch.Tensor, views: dict):
        self.layer, self.n_experts, self.buf, self.views = layer, n_experts, buf, views

    @property
    def nbytes(self) -> int:
        return self.buf.numel()

    def source(self, layer: int, expert: int, which: str):
        if layer != self.layer:
            raise KeyError(f"layer {layer} is not resident (this table holds layer {self.layer})")
        return self.views[(expert, which)]
