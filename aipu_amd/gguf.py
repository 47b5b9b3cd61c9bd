"""GGUF v3 tensor ingestion into device buffers in ggml block layout.

The hot-path kernels take weights exactly as a GGUF file stores them (ggml row blocks,
``ne = [K, N]`` or ``[K, N, E]`` for fused expert stacks), so ingestion is a bounded
header parse plus byte copies -- no repacking.

Reference counterparts:

* ``read_gguf`` / ``write_gguf`` -- the in-memory GGUF v3 codec of
  ``tools/ckpt_pack_q4k.py:104-182`` (same arguments and return values; the writer is used
  to make synthetic files).
* the ggml type table -- ``tools/ckpt_pack_q4k.py:58-68`` (F32, F16, Q8_0, Q4_K, Q6_K), plus
  BF16 and the other ggml block sizes so that headers of real checkpoints parse (only the
  types the kernels read can be uploaded).
* ``read_header`` -- the bounded streaming header parser of
  ``tools/provision_image.py:110-205``: seek + read field by field, KV values other than the
  alignment and name skipped without being held, the tensor blob never touched.
* ``classify`` -- the resident-hot / streamed-expert rule of ``tools/provision_image.py:60-83``.

``GGUFFile.upload`` copies a tensor into a device ``torch.uint8`` buffer through a pinned
staging buffer of bounded size (default 64 MiB), memory-mapping the file, so a checkpoint of
any size streams with O(staging) host memory.
"""
from __future__ import annotations

import os
import struct
from dataclasses import dataclass, field

import numpy as np

GGUF_MAGIC = 0x46554747          # b"GGUF" read as a little-endian uint32
GGUF_VERSION = 3
DEFAULT_ALIGNMENT = 32

GGML_F32, GGML_F16, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K, GGML_BF16 = 0, 1, 8, 12, 14, 30

# ggml type id -> (name, weights per block, bytes per block)
GGML_TYPES = {
    0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20),
    6: ("Q5_0", 32, 22), 7: ("Q5_1", 32, 24), 8: ("Q8_0", 32, 34), 9: ("Q8_1", 32, 36),
    10: ("Q2_K", 256, 84), 11: ("Q3_K", 256, 110), 12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176),
    14: ("Q6_K", 256, 210), 15: ("Q8_K", 256, 292), 24: ("I8", 1, 1), 25: ("I16", 1, 2),
    26: ("I32", 1, 4), 27: ("I64", 1, 8), 28: ("F64", 1, 8), 30: ("BF16", 1, 2),
}
TYPE_NAME = {t: v[0] for t, v in GGML_TYPES.items()}
BLOCK = {t: (v[1], v[2]) for t, v in GGML_TYPES.items()}

# Types the GEMV / MoE / LM-head kernels read directly (same ids in include/aipu_q4k.h).
KERNEL_TYPES = (GGML_Q4_K, GGML_Q6_K, GGML_Q8_0, GGML_F16, GGML_BF16)

# KV value types: id -> struct format (fixed width); 8 = string, 9 = array
_KV_FIXED = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?",
             10: "<Q", 11: "<q", 12: "<d"}
KV_UINT32, KV_STRING, KV_ARRAY = 4, 8, 9


class GGUFError(ValueError):
    pass


def tnbytes(ttype, nelem):
    """Bytes of a tensor of `nelem` weights of ggml type `ttype` (whole blocks only)."""
    if ttype not in BLOCK:
        raise GGUFError(f"unknown ggml type {ttype}")
    epb, bpb = BLOCK[ttype]
    if nelem % epb:
        raise GGUFError(f"{nelem} weights are not a whole number of {TYPE_NAME[ttype]} blocks of {epb}")
    return nelem // epb * bpb


def _nelem(dims):
    n = 1
    for d in dims:
        n *= int(d)
    return n


def classify(name):
    """'streamed_expert' for fused routed-expert stacks (ggml's ``_exps`` suffix and the
    ``experts.`` / ``.expert.`` spellings of other converters), else 'resident_hot'."""
    n = name.lower()
    expert = ("_exps" in n or ".exps." in n or n.endswith(".exps.weight") or "experts." in n or ".expert." in n)
    return "streamed_expert" if expert else "resident_hot"


# ------------------------------------------------------------------ writer
def _str(s):
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def write_gguf(tensors, arch="glm", alignment=DEFAULT_ALIGNMENT):
    """GGUF v3 bytes for `tensors` = [(name, ggml_type, dims_ne, raw_bytes)], dims in ggml ne
    order (dims[0] fastest).  Metadata: general.architecture, general.alignment,
    general.quantization_version = 2.  Each tensor's data starts on an `alignment` boundary
    of the data section, which itself starts aligned."""
    kv = (_str("general.architecture") + struct.pack("<I", KV_STRING) + _str(arch)
          + _str("general.alignment") + struct.pack("<II", KV_UINT32, alignment)
          + _str("general.quantization_version") + struct.pack("<II", KV_UINT32, 2))
    head = struct.pack("<IIQQ", GGUF_MAGIC, GGUF_VERSION, len(tensors), 3) + kv
    infos, blob = [], bytearray()
    for name, ttype, dims, raw in tensors:
        want = tnbytes(ttype, _nelem(dims))
        if len(raw) != want:
            raise GGUFError(f"{name}: {len(raw)} bytes given, {want} needed for {TYPE_NAME[ttype]} {list(dims)}")
        info = _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", int(d)) for d in dims)
        infos.append(info + struct.pack("<IQ", ttype, len(blob)))
        blob += bytes(raw)
        blob += b"\0" * (-len(blob) % alignment)
    pre = head + b"".join(infos)
    return pre + b"\0" * (-len(pre) % alignment) + bytes(blob)


# ------------------------------------------------------------------ readers
class _Cursor:
    """Sequential little-endian reads from a bytes-like object or a binary file."""

    def __init__(self, src):
        self.buf = src if isinstance(src, (bytes, bytearray, memoryview)) else None
        self.fh = None if self.buf is not None else src
        self.off = 0

    def read(self, n):
        if self.buf is not None:
            b = bytes(self.buf[self.off:self.off + n])
        else:
            b = self.fh.read(n)
        if len(b) != n:
            raise GGUFError("truncated GGUF header")
        self.off += n
        return b

    def skip(self, n):
        if self.buf is not None:
            if self.off + n > len(self.buf):
                raise GGUFError("truncated GGUF header")
        else:
            self.fh.seek(n, os.SEEK_CUR)
        self.off += n

    def take(self, fmt):
        return struct.unpack(fmt, self.read(struct.calcsize(fmt)))[0]

    def string(self):
        return self.read(self.take("<Q")).decode("utf-8", "replace")

    def value(self, vtype, keep=True):
        """One KV value; with keep=False it is skipped (arrays of fixed-width elements by a
        single seek) and None returned."""
        if vtype in _KV_FIXED:
            fmt = _KV_FIXED[vtype]
            if not keep:
                self.skip(struct.calcsize(fmt))
                return None
            return self.take(fmt)
        if vtype == KV_STRING:
            if not keep:
                self.skip(self.take("<Q"))
                return None
            return self.string()
        if vtype == KV_ARRAY:
            etype, n = self.take("<I"), self.take("<Q")
            if not keep and etype in _KV_FIXED:
                self.skip(struct.calcsize(_KV_FIXED[etype]) * n)
                return None
            vals = [self.value(etype, keep) for _ in range(n)]
            return vals if keep else None
        raise GGUFError(f"unknown GGUF value type {vtype}")


@dataclass
class TensorInfo:
    name: str
    ggml_type: int
    dims: list           # ggml ne order: dims[0] = K (fastest), dims[1] = N, dims[2] = E
    offset: int          # absolute file offset of the first byte
    nbytes: int

    @property
    def type_name(self):
        return TYPE_NAME.get(self.ggml_type, f"TYPE_{self.ggml_type}")

    @property
    def kind(self):
        return classify(self.name)


@dataclass
class GGUFHeader:
    version: int
    alignment: int
    data_start: int
    meta: dict = field(default_factory=dict)
    tensors: list = field(default_factory=list)

    def by_name(self):
        return {t.name: t for t in self.tensors}


def _parse(cur, keep_all_meta, want=("general.alignment", "general.name", "general.architecture")):
    magic = cur.take("<I")
    if magic != GGUF_MAGIC:
        raise GGUFError(f"bad GGUF magic {magic:#x}")
    version = cur.take("<I")
    if version != GGUF_VERSION:
        raise GGUFError(f"unsupported GGUF version {version}")
    n_tensors, n_kv = cur.take("<Q"), cur.take("<Q")
    meta = {}
    for _ in range(n_kv):
        key = cur.string()
        vtype = cur.take("<I")
        keep = keep_all_meta or key in want
        val = cur.value(vtype, keep)
        if keep:
            meta[key] = val
    raw_infos = []
    for _ in range(n_tensors):
        name = cur.string()
        ndim = cur.take("<I")
        dims = [cur.take("<Q") for _ in range(ndim)]
        raw_infos.append((name, dims, cur.take("<I"), cur.take("<Q")))
    align = meta.get("general.alignment", DEFAULT_ALIGNMENT)
    if not isinstance(align, int) or align <= 0:
        raise GGUFError(f"bad general.alignment {align!r}")
    data_start = cur.off + (-cur.off % align)
    infos = [TensorInfo(n, t, d, data_start + o, tnbytes(t, _nelem(d))) for n, d, t, o in raw_infos]
    return GGUFHeader(version, align, data_start, meta, infos)


def read_gguf(buf):
    """Parse GGUF bytes -> (metadata dict, {name: (ggml_type, dims, raw bytes)})."""
    hdr = _parse(_Cursor(memoryview(buf)), keep_all_meta=True)
    out = {}
    for t in hdr.tensors:
        if t.offset + t.nbytes > len(buf):
            raise GGUFError(f"{t.name}: data runs past the end of the file")
        out[t.name] = (t.ggml_type, list(t.dims), bytes(buf[t.offset:t.offset + t.nbytes]))
    return hdr.meta, out


def read_header(path):
    """Stream only the header of a GGUF file (bounded memory, no tensor data read)."""
    with open(path, "rb") as fh:
        hdr = _parse(_Cursor(fh), keep_all_meta=False)
        size = os.fstat(fh.fileno()).st_size
    for t in hdr.tensors:
        if t.offset + t.nbytes > size:
            raise GGUFError(f"{t.name}: data runs past the end of the file")
    return hdr


# ------------------------------------------------------------------ device upload
@dataclass
class DeviceTensor:
    """One GGUF tensor resident on the device: raw ggml blocks as a uint8 tensor."""
    name: str
    ggml_type: int
    dims: list
    data: object          # torch.uint8 tensor on the device

    @property
    def K(self):
        return int(self.dims[0])

    @property
    def N(self):
        return int(self.dims[1]) if len(self.dims) > 1 else 1

    @property
    def E(self):
        return int(self.dims[2]) if len(self.dims) > 2 else 1

    def expert(self, e):
        """Blocks of expert e of a fused [K, N, E] stack (a view, no copy)."""
        if not 0 <= e < self.E:
            raise IndexError(f"expert {e} of {self.E}")
        per = self.data.numel() // self.E
        return self.data[e * per:(e + 1) * per]

    def as_bf16_rows(self):
        """A BF16 / F16 matrix as a [N, K] 16-bit tensor view (for the LM head)."""
        import torch
        if self.ggml_type == GGML_BF16:
            return self.data.view(torch.bfloat16).view(self.N, self.K)
        if self.ggml_type == GGML_F16:
            return self.data.view(torch.float16).view(self.N, self.K)
        raise GGUFError(f"{self.name} is {TYPE_NAME[self.ggml_type]}, not a 16-bit float matrix")


class GGUFFile:
    """A GGUF checkpoint on disk: header parsed once, tensors uploaded on request."""

    def __init__(self, path):
        self.path = path
        self.header = read_header(path)
        self._infos = self.header.by_name()
        self._mm = None

    @property
    def tensors(self):
        return self.header.tensors

    def info(self, name):
        try:
            return self._infos[name]
        except KeyError:
            raise KeyError(f"{name} is not in {self.path}") from None

    def _map(self):
        if self._mm is None:
            self._mm = np.memmap(self.path, dtype=np.uint8, mode="r")
        return self._mm

    def host_bytes(self, name):
        """The tensor's bytes as a read-only memory-mapped numpy view."""
        t = self.info(name)
        return self._map()[t.offset:t.offset + t.nbytes]

    def upload(self, name, device="cuda", staging_bytes=64 << 20, out=None):
        """Copy one tensor into a device uint8 buffer (or `out`), through a pinned staging
        buffer of at most `staging_bytes`, and return a DeviceTensor."""
        import torch
        t = self.info(name)
        if t.ggml_type not in KERNEL_TYPES and t.ggml_type != GGML_F32:
            raise GGUFError(f"{name}: {t.type_name} is not a type the kernels read")
        dst = out if out is not None else torch.empty(t.nbytes, dtype=torch.uint8, device=device)
        if dst.numel() != t.nbytes or dst.dtype != torch.uint8:
            raise GGUFError(f"{name}: destination must be {t.nbytes} uint8")
        src = self.host_bytes(name)
        step = max(16, min(staging_bytes, t.nbytes))
        # two pinned buffers: one fills from the file while the other's copy is in flight
        stages = [torch.empty(step, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
        done = [None, None]
        stream = torch.cuda.current_stream(dst.device)
        for i, o in enumerate(range(0, t.nbytes, step)):
            k = i & 1
            n = min(step, t.nbytes - o)
            if done[k] is not None:
                done[k].synchronize()          # that buffer's previous copy has finished
            stages[k][:n].numpy()[:] = src[o:o + n]
            dst[o:o + n].copy_(stages[k][:n], non_blocking=True)
            done[k] = torch.cuda.Event()
            done[k].record(stream)
        stream.synchronize()
        return DeviceTensor(name, t.ggml_type, list(t.dims), dst)

    def upload_all(self, device="cuda", names=None, kind=None, staging_bytes=64 << 20):
        """Upload every tensor (or those in `names`, or of one classify() kind)."""
        out = {}
        for t in self.tensors:
            if names is not None and t.name not in names:
                continue
            if kind is not None and t.kind != kind:
                continue
            out[t.name] = self.upload(t.name, device, staging_bytes)
        return out

    def close(self):
        self._mm = None


__all__ = [
    "GGUF_MAGIC", "GGUF_VERSION", "GGML_F32", "GGML_F16", "GGML_Q8_0", "GGML_Q4_K", "GGML_Q6_K", "GGML_BF16",
    "GGML_TYPES", "TYPE_NAME", "BLOCK", "KERNEL_TYPES", "GGUFError", "tnbytes", "classify", "write_gguf",
    "read_gguf", "read_header", "TensorInfo", "GGUFHeader", "DeviceTensor", "GGUFFile",
]
