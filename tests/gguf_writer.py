"""A minimal GGUF v3 writer for the reader's tests, written from the public
GGUF layout independently of the reader (little-endian; string = u64 length
+ bytes; metadata entry = key, u32 value type, value; array = u32 element
type, u64 count, elements; tensor info = name, u32 n_dims, u64 dims, u32 type,
u64 offset; tensor data after padding the header to the alignment)."""
import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(vtype, v):
    if vtype in _FMT:
        return struct.pack(_FMT[vtype], v)
    if vtype == STRING:
        return _str(v)
    if vtype == ARRAY:
        etype, items = v
        out = struct.pack("<IQ", etype, len(items))
        for it in items:
            out += _value(etype, it)
        return out
    raise ValueError(vtype)


def gguf_bytes(kv=(), tensors=(), alignment=None, version=3, magic=b"GGUF"):
    """kv: [(key, vtype, value)] (arrays: value = (elem type, items)); tensors:
    [(name, dims in GGUF order, ggml type id, raw bytes)].  Tensor data is
    laid out in order, each start padded to the alignment."""
    align = alignment or 32
    kv = list(kv)
    if alignment is not None:
        kv.append(("general.alignment", U32, alignment))
    head = magic + struct.pack("<IQQ", version, len(tensors), len(kv))
    for key, vtype, v in kv:
        head += _str(key) + struct.pack("<I", vtype) + _value(vtype, v)
    data = b""
    for name, dims, ttype, raw in tensors:
        off = (len(data) + align - 1) // align * align
        data = data.ljust(off, b"\0")
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ttype, off)
        data += raw
    pad = (len(head) + align - 1) // align * align
    return head.ljust(pad, b"\0") + data


def write_gguf(path, **kw):
    blob = gguf_bytes(**kw)
    with open(path, "wb") as f:
        f.write(blob)
    return str(path)
