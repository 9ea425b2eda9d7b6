"""GGUF wire-byte loading on top of the library's native reader (kq_gguf.h).

Mirrors the reference's GGUF entry points:
  load_gguf(path, zero_copy)      kq.load_gguf as called at gmlx/loader.py:124
                                  (returns arrays, codecs, metadata, shapes)
  load_gguf_wire_bytes(path, ...) gmlx/loader.py:92-142 (split shards merged)
  scan_gguf(path, ...)            gmlx/headerscan.py:122-176 (metadata and
                                  tensor table, large arrays skipped,
                                  truncation detected)
  find_split_shards(path)         gmlx/preflight.py:75-101
  split_fused_gate_up, qk_permute_wire, qk_permute_wire_inverse
                                  gmlx/transforms.py:132-184

K-quant tensors come back as uint8 wire bytes shaped (..., rows, row_bytes)
(the GGUF dims reversed, the innermost one in bytes), exactly the rows the
matmul kernels consume, with the vestigial `<prefix>.scales` placeholder the
reference's modules expect; float and integer tensors come back in their own
dtype.  With zero_copy the CPU tensors view the file's read-only mapping
(kept alive by the tensors); `device=` copies each tensor to that device.
"""
from __future__ import annotations

import ctypes
import os
import re
import struct
from dataclasses import dataclass

from ._lib import KQ_ERR_BAD_FORMAT, KQ_ERR_IO, KQ_OK, lib

# GGML type id -> name (the public GGML type table)
GGML_TYPES = {
    0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0", 9: "Q8_1",
    10: "Q2_K", 11: "Q3_K", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 15: "Q8_K", 16: "IQ2_XXS",
    17: "IQ2_XS", 18: "IQ3_XXS", 19: "IQ1_S", 20: "IQ4_NL", 21: "IQ3_S", 22: "IQ2_S", 23: "IQ4_XS",
    24: "I8", 25: "I16", 26: "I32", 27: "I64", 28: "F64", 29: "IQ1_M", 30: "BF16", 34: "TQ1_0",
    35: "TQ2_0", 39: "MXFP4",
}
# unquantized types: loaded in their own dtype
_PLAIN = {"F32": "float32", "F16": "float16", "BF16": "bfloat16", "F64": "float64",
          "I8": "int8", "I16": "int16", "I32": "int32", "I64": "int64"}

DEFAULT_ARRAY_LIMIT = 2048
SPLIT_SHARD_RE = re.compile(r"-(\d{5})-of-(\d{5})\.gguf$")

# GGUF metadata value types
_SCALARS = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q",
            12: "<d"}
_STRING, _ARRAY = 8, 9


class GGUFError(ValueError):
    """A malformed or unreadable GGUF file."""


@dataclass(frozen=True)
class TensorInfo:
    name: str
    shape: tuple          # GGUF order: shape[0] is the row length (varies fastest)
    type_id: int
    type_name: str
    offset: int           # relative to the data section
    nbytes: int


@dataclass(frozen=True)
class HeaderScan:
    path: str
    version: int
    kv: dict
    skipped: dict         # key -> element count of arrays over the limit
    tensors: list
    n_tensors: int
    data_offset: int
    expected_size: int    # data_offset + end of the last tensor; 0 without tensors
    size: int             # actual file size
    truncated: bool


def _open_error(path, rc):
    if rc == KQ_ERR_IO:
        return OSError(f"{path}: cannot open or map the file")
    if rc == KQ_ERR_BAD_FORMAT:
        return GGUFError(f"{path}: not a valid GGUF v2/v3 file")
    return GGUFError(f"{path}: {lib().kq_strerror(rc).decode()}")


def _read_values(addr, etype, count):
    """Decode `count` values of GGUF type `etype` at address `addr`; returns
    (values, bytes consumed)."""
    fmt = _SCALARS.get(etype)
    if fmt is not None:
        size = struct.calcsize(fmt)
        raw = ctypes.string_at(addr, size * count)
        vals = [v[0] for v in struct.iter_unpack(fmt, raw)] if count else []
        return vals, size * count
    out, off = [], 0
    for _ in range(count):
        if etype == _STRING:
            (n,) = struct.unpack("<Q", ctypes.string_at(addr + off, 8))
            out.append(ctypes.string_at(addr + off + 8, n).decode("utf-8", errors="replace"))
            off += 8 + n
        elif etype == _ARRAY:
            et, n = struct.unpack("<IQ", ctypes.string_at(addr + off, 12))
            vals, used = _read_values(addr + off + 12, et, n)
            out.append(vals)
            off += 12 + used
        else:
            raise GGUFError(f"unknown GGUF value type {etype}")
    return out, off


class GGUFFile:
    """An open GGUF file: header, metadata and tensor table parsed by the
    native reader; tensor bytes are read in place from the mapping."""

    def __init__(self, path):
        self.path = os.path.expanduser(str(path))
        L = lib()
        h = ctypes.c_void_p()
        rc = L.kq_gguf_open(self.path.encode(), ctypes.byref(h))
        if rc != KQ_OK:
            raise _open_error(self.path, rc)
        self._h = h
        v = ctypes.c_uint32()
        nt, nk, do, al, fs, es = (ctypes.c_int64() for _ in range(6))
        L.kq_gguf_header(h, ctypes.byref(v), ctypes.byref(nt), ctypes.byref(nk), ctypes.byref(do),
                         ctypes.byref(al), ctypes.byref(fs), ctypes.byref(es))
        self.version, self.n_tensors, self.n_kv = v.value, nt.value, nk.value
        self.data_offset, self.alignment, self.size, self.expected_size = do.value, al.value, fs.value, es.value
        self.truncated = bool(self.expected_size and self.size < self.expected_size)
        self._tensors = None
        self._views = False

    # ---- lifetime
    def close(self, _final=False):
        """Unmap the file, unless zero-copy tensors still view it: then the
        mapping is released with the last of them."""
        if getattr(self, "_views", False) and not _final:
            return
        if getattr(self, "_h", None) is not None and self._h.value:
            lib().kq_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close(_final=True)  # no view is left: they hold a reference to this object
        except Exception:
            pass

    def _handle(self):
        if self._h is None:
            raise ValueError(f"{self.path}: GGUF file is closed")
        return self._h

    # ---- metadata
    def metadata(self, array_limit=None):
        """(kv, skipped): every metadata entry decoded; arrays longer than
        `array_limit` are not decoded and appear in `skipped` with their
        element count."""
        L, h = lib(), self._handle()
        kv, skipped = {}, {}
        key, kl, t, et, cnt, data = (ctypes.c_void_p(), ctypes.c_int64(), ctypes.c_uint32(), ctypes.c_uint32(),
                                     ctypes.c_int64(), ctypes.c_void_p())
        for i in range(self.n_kv):
            L.kq_gguf_kv(h, i, ctypes.byref(key), ctypes.byref(kl), ctypes.byref(t), ctypes.byref(et),
                         ctypes.byref(cnt), ctypes.byref(data))
            name = ctypes.string_at(key.value, kl.value).decode("utf-8", errors="replace")
            if t.value == _STRING:
                kv[name] = ctypes.string_at(data.value, cnt.value).decode("utf-8", errors="replace") \
                    if cnt.value else ""
            elif t.value == _ARRAY:
                if array_limit is not None and cnt.value > array_limit:
                    skipped[name] = cnt.value
                else:
                    kv[name] = _read_values(data.value, et.value, cnt.value)[0] if cnt.value else []
            else:
                kv[name] = _read_values(data.value, t.value, 1)[0][0]
        return kv, skipped

    # ---- tensors
    @property
    def tensors(self):
        if self._tensors is None:
            L, h = lib(), self._handle()
            out = []
            name, nl, nd, ty, off, nb, data = (ctypes.c_void_p(), ctypes.c_int64(), ctypes.c_uint32(),
                                               ctypes.c_uint32(), ctypes.c_int64(), ctypes.c_int64(),
                                               ctypes.c_void_p())
            dims = (ctypes.c_int64 * 4)()
            for i in range(self.n_tensors):
                L.kq_gguf_tensor(h, i, ctypes.byref(name), ctypes.byref(nl), ctypes.byref(nd), dims,
                                 ctypes.byref(ty), ctypes.byref(off), ctypes.byref(nb), ctypes.byref(data))
                out.append(TensorInfo(ctypes.string_at(name.value, nl.value).decode("utf-8", errors="replace"),
                                      tuple(int(dims[d]) for d in range(nd.value)), int(ty.value),
                                      GGML_TYPES[int(ty.value)], int(off.value), int(nb.value)))
            self._tensors = out
        return self._tensors

    def tensor_address(self, index):
        """Address of tensor `index`'s bytes in the mapping (None past the end
        of a truncated file)."""
        data = ctypes.c_void_p()
        lib().kq_gguf_tensor(self._handle(), index, None, None, None, None, None, None, None, ctypes.byref(data))
        return data.value

    def tensor(self, index, zero_copy=True, device=None):
        """Tensor `index` as torch: wire bytes (..., rows, row_bytes) for a
        quantized type, else its own dtype; dims in torch order (the GGUF
        dims reversed)."""
        import numpy as np
        import torch
        info = self.tensors[index]
        addr = self.tensor_address(index)
        if addr is None:
            raise GGUFError(f"{self.path}: tensor {info.name} lies past the end of the file (truncated)")
        buf = (ctypes.c_uint8 * info.nbytes).from_address(addr)
        buf._gguf_keepalive = self  # the mapping lives as long as any view of it
        raw = np.frombuffer(buf, dtype=np.uint8)
        dims = list(reversed(info.shape))
        plain = _PLAIN.get(info.type_name)
        if plain is None:
            shape = dims[:-1] + [info.nbytes // max(1, _rows(dims))]
            t = torch.from_numpy(raw).view(*shape) if info.nbytes else torch.empty(shape, dtype=torch.uint8)
        elif plain == "bfloat16":
            t = torch.from_numpy(raw).view(torch.bfloat16).view(*dims)
        else:
            t = torch.from_numpy(raw.view(np.dtype(plain))).view(*dims)
        if not zero_copy:
            t = t.clone()
        if device is not None:
            t = t.to(device)
        if zero_copy and device is None:
            self._views = True  # t views the mapping (read-only memory: do not write to it)
        return t


def _rows(dims_torch):
    n = 1
    for d in dims_torch[:-1]:
        n *= d
    return n


def codec_name(type_name):
    """The codec string the reference's modules use for a quantized type
    ("q4_k", "iq2_xxs", ...); None for float / integer types."""
    return None if type_name in _PLAIN else type_name.lower()


def scan_gguf(path, *, include_tensors=True, array_limit=DEFAULT_ARRAY_LIMIT):
    """Metadata and tensor table without touching tensor data
    (gmlx/headerscan.py:122-176): arrays over `array_limit` elements are
    skipped and counted; `truncated` when the file is shorter than the tensor
    table implies.  Raises GGUFError on a malformed header."""
    with GGUFFile(path) as g:
        kv, skipped = g.metadata(array_limit)
        tensors = list(g.tensors) if include_tensors else []
        return HeaderScan(path=g.path, version=g.version, kv=kv, skipped=skipped, tensors=tensors,
                          n_tensors=g.n_tensors, data_offset=g.data_offset if include_tensors else 0,
                          expected_size=g.expected_size if include_tensors else 0, size=g.size,
                          truncated=g.truncated if include_tensors else False)


def load_gguf(path, zero_copy=True, device=None):
    """kq.load_gguf: (arrays, codecs, meta, shapes) of one GGUF file.

    arrays: name -> tensor (quantized: uint8 wire rows, plus a `.scales`
    placeholder per quantized weight); codecs: name -> codec string of every
    quantized tensor; meta: every metadata entry decoded; shapes: name ->
    logical shape in GGUF order."""
    import torch
    g = GGUFFile(path)
    if g.truncated:
        g.close()
        raise GGUFError(f"{path}: truncated ({g.size} of {g.expected_size} bytes)")
    meta, _ = g.metadata(None)
    arrays, codecs, shapes = {}, {}, {}
    for i, info in enumerate(g.tensors):
        arrays[info.name] = g.tensor(i, zero_copy=zero_copy, device=device)
        shapes[info.name] = info.shape
        c = codec_name(info.type_name)
        if c is not None:
            codecs[info.name] = c
            prefix = info.name[:-len(".weight")] if info.name.endswith(".weight") else info.name
            arrays[prefix + ".scales"] = torch.zeros((1,), dtype=torch.uint8, device=device)
    g.close()  # kept mapped while zero-copy tensors view it
    return arrays, codecs, meta, shapes


def find_split_shards(gguf_path):
    """The shard files of a model, in load order.

    A split GGUF names its shards `<stem>-<i>-of-<n>.gguf` (five-digit
    i = 1..n, the split naming of gmlx/preflight.py:75-101): any one shard's
    path yields all n, in index order.  Any other path is a single-file model
    and comes back alone.  Every shard must exist -- a missing one would leave
    its tensors unloaded -- so the absent ones are reported together."""
    path = os.path.expanduser(str(gguf_path))
    folder, name = os.path.split(path)
    m = SPLIT_SHARD_RE.search(name)
    if m is None:
        return [path]
    stem, count = name[:m.start()], int(m.group(2))
    shards = [os.path.join(folder, f"{stem}-{i:05d}-of-{count:05d}.gguf") for i in range(1, count + 1)]
    absent = [i + 1 for i, p in enumerate(shards) if not os.path.isfile(p)]
    if absent:
        listed = ", ".join(str(i) for i in absent[:8]) + (" ..." if len(absent) > 8 else "")
        raise FileNotFoundError(f"split GGUF {stem!r} is incomplete: {len(absent)}/{count} shard(s) absent "
                                f"(index {listed}) in {folder or '.'}")
    return shards


def load_gguf_wire_bytes(gguf_path, zero_copy=True, shards=None, expect_quant=True, device=None):
    """gmlx/loader.py:92-142: every shard loaded and merged; metadata and
    shapes from the first shard.  Returns (arrays, codecs, arch, meta,
    shapes)."""
    import warnings
    shards = shards if shards is not None else find_split_shards(gguf_path)
    arrays, codecs, meta, shapes = {}, {}, {}, {}
    for i, shard in enumerate(shards):
        a, c, m, s = load_gguf(shard, zero_copy=zero_copy, device=device)
        arrays.update(a)
        codecs.update(c)
        shapes.update(s)
        if i == 0:
            meta = m
    if expect_quant and not codecs:
        warnings.warn("no quantized tensors found - is this actually a K-quant GGUF?")
    return arrays, codecs, meta.get("general.architecture"), meta, shapes


# ---------------------------------------------------------------- transforms

def split_fused_gate_up(w):
    """(gate, up) halves of a fused expert gate|up wire tensor
    (n_experts, 2 * inter, row_bytes), each made row-contiguous."""
    if w.dim() != 3:
        raise ValueError(f"expected a 3-D fused expert tensor, got shape {tuple(w.shape)}")
    half = w.shape[-2] // 2
    return w[..., :half, :].contiguous(), w[..., half:, :].contiguous()


def qk_permute_wire(w, n_head):
    """Undo llama.cpp's Q/K row permutation (rows regrouped per head from
    (2, D/2) to (D/2, 2) order) on wire rows."""
    n_out = w.shape[0]
    hd = n_out // n_head
    return w.reshape(n_head, hd // 2, 2, *w.shape[1:]).transpose(1, 2).reshape(n_out, *w.shape[1:])


def qk_permute_wire_inverse(w, n_head):
    """Apply llama.cpp's Q/K row permutation (inverse of qk_permute_wire)."""
    n_out = w.shape[0]
    hd = n_out // n_head
    return w.reshape(n_head, 2, hd // 2, *w.shape[1:]).transpose(1, 2).reshape(n_out, *w.shape[1:])
