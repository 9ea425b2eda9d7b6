"""GGUF wire-byte reader (include/kq_gguf.h through gmlx_amd.gguf): metadata
of every value type, large arrays skipped, the tensor table and tensor bytes,
truncation, malformed headers, alignment, split shards and the wire-row
transforms.  Mirrors the reference's header-scan tests
(tests/test_headerscan.py: KV parity, skipped arrays, tensor table,
truncation, bad magic) on files written by tests/gguf_writer.py, an
independent writer of the public GGUF layout."""
import numpy as np
import pytest
import torch

from gguf_writer import (ARRAY, BOOL, F32, F64, I8, I16, I32, I64, STRING, U8, U16, U32, U64, gguf_bytes,
                         write_gguf)
from gmlx_amd import gguf
from oracle import kquant as okq

BASIC_KV = [
    ("general.architecture", STRING, "llama"),
    ("general.name", STRING, "scan-fixture"),
    ("llama.block_count", U32, 2),
    ("llama.context_length", U32, 4096),
    ("llama.rope.freq_base", F32, 10000.0),
    ("tokenizer.ggml.add_bos_token", BOOL, True),
    ("llama.small_ints", ARRAY, (I32, [1, 2, 3])),
    ("llama.small_floats", ARRAY, (F32, [0.5, 1.5])),
    ("llama.small_bools", ARRAY, (BOOL, [True, False, True])),
    ("llama.small_strs", ARRAY, (STRING, ["a", "bb", "ccc"])),
]


def _rng_wire(rng, codec, rows, k):
    w = rng.normal(0.0, 0.02, size=(rows, k)).astype(np.float32)
    return okq.quantize(w, codec)


def _fixture(tmp_path, rng, big_arrays=False, alignment=None):
    kv = list(BASIC_KV)
    if big_arrays:
        kv.append(("tokenizer.ggml.tokens", ARRAY, (STRING, [f"tok{i}" for i in range(5000)])))
        kv.append(("tokenizer.ggml.token_type", ARRAY, (I32, [1] * 5000)))
    f32 = rng.normal(size=(32, 64)).astype(np.float32)            # torch shape (32, 64): GGUF dims (64, 32)
    f16 = rng.normal(size=(64, 64)).astype(np.float16)
    bf16 = torch.randn(8, 32, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    q4 = _rng_wire(rng, "q4_k", 8, 512)                            # 8 rows of 2 blocks
    q6 = _rng_wire(rng, "q6_k", 4, 256)
    iq2 = _rng_wire(rng, "iq2_xxs", 3, 768)
    experts = _rng_wire(rng, "q4_k", 2 * 6, 256).reshape(2, 6, 144)  # 2 experts x 6 rows
    tensors = [
        ("token_embd.weight", (64, 32), 0, f32.tobytes()),
        ("blk.0.attn_q.weight", (64, 64), 1, f16.tobytes()),
        ("blk.0.attn_norm.weight", (32, 8), 30, bf16.view(torch.int16).numpy().tobytes()),
        ("blk.0.attn_k.weight", (512, 8), 12, q4.tobytes()),
        ("blk.0.attn_v.weight", (256, 4), 14, q6.tobytes()),
        ("blk.0.ffn_down.weight", (768, 3), 16, iq2.tobytes()),
        ("blk.0.ffn_gate_exps.weight", (256, 6, 2), 12, experts.tobytes()),
    ]
    path = write_gguf(tmp_path / "m.gguf", kv=kv, tensors=tensors, alignment=alignment)
    return path, dict(f32=f32, f16=f16, bf16=bf16, q4=q4, q6=q6, iq2=iq2, experts=experts)


def test_kv_parity(tmp_path):
    p, _ = _fixture(tmp_path, np.random.default_rng(0))
    scan = gguf.scan_gguf(p, include_tensors=False)
    assert scan.version == 3
    assert scan.kv["general.architecture"] == "llama"
    assert scan.kv["general.name"] == "scan-fixture"
    assert scan.kv["llama.block_count"] == 2
    assert scan.kv["llama.rope.freq_base"] == pytest.approx(10000.0)
    assert scan.kv["tokenizer.ggml.add_bos_token"] is True
    assert scan.kv["llama.small_ints"] == [1, 2, 3]
    assert scan.kv["llama.small_floats"] == pytest.approx([0.5, 1.5])
    assert scan.kv["llama.small_bools"] == [True, False, True]
    assert scan.kv["llama.small_strs"] == ["a", "bb", "ccc"]
    assert scan.skipped == {}


def test_every_value_type(tmp_path):
    kv = [("u8", U8, 255), ("i8", I8, -128), ("u16", U16, 65535), ("i16", I16, -32768), ("u32", U32, 2 ** 32 - 1),
          ("i32", I32, -2 ** 31), ("f32", F32, 1.25), ("bool", BOOL, False), ("str", STRING, "héllo"),
          ("empty", STRING, ""), ("u64", U64, 2 ** 64 - 1), ("i64", I64, -2 ** 63), ("f64", F64, 2.0 ** -40),
          ("nested", ARRAY, (ARRAY, [(U16, [1, 2]), (U16, []), (U16, [7])])),
          ("empty_arr", ARRAY, (F64, []))]
    p = write_gguf(tmp_path / "kv.gguf", kv=kv)
    got = gguf.scan_gguf(p).kv
    want = {k: v for k, _, v in kv}
    want["nested"] = [[1, 2], [], [7]]
    want["empty_arr"] = []
    assert got == want


def test_large_arrays_skipped_not_read(tmp_path):
    p, _ = _fixture(tmp_path, np.random.default_rng(0), big_arrays=True)
    scan = gguf.scan_gguf(p, include_tensors=False)
    assert scan.skipped == {"tokenizer.ggml.tokens": 5000, "tokenizer.ggml.token_type": 5000}
    assert "tokenizer.ggml.tokens" not in scan.kv
    assert scan.kv["llama.block_count"] == 2    # entries after the skipped arrays parse
    full = gguf.scan_gguf(p, include_tensors=False, array_limit=10 ** 6)
    assert full.kv["tokenizer.ggml.tokens"][4999] == "tok4999" and full.skipped == {}


def test_tensor_table_and_bytes(tmp_path):
    p, ref = _fixture(tmp_path, np.random.default_rng(1))
    scan = gguf.scan_gguf(p)
    by = {t.name: t for t in scan.tensors}
    assert by["token_embd.weight"].shape == (64, 32) and by["token_embd.weight"].type_name == "F32"
    assert by["blk.0.attn_k.weight"].type_name == "Q4_K" and by["blk.0.attn_k.weight"].nbytes == 8 * 2 * 144
    assert by["blk.0.ffn_down.weight"].type_name == "IQ2_XXS" and by["blk.0.ffn_down.weight"].nbytes == 3 * 3 * 66
    assert all(t.offset % 32 == 0 for t in scan.tensors) and scan.data_offset % 32 == 0
    assert scan.expected_size == scan.size and not scan.truncated
    arrays, codecs, meta, shapes = gguf.load_gguf(p)
    assert codecs == {"blk.0.attn_k.weight": "q4_k", "blk.0.attn_v.weight": "q6_k",
                      "blk.0.ffn_down.weight": "iq2_xxs", "blk.0.ffn_gate_exps.weight": "q4_k"}
    assert meta["general.architecture"] == "llama"
    assert shapes["blk.0.attn_k.weight"] == (512, 8)
    assert np.array_equal(arrays["token_embd.weight"].numpy(), ref["f32"])
    assert arrays["blk.0.attn_q.weight"].dtype == torch.float16
    assert np.array_equal(arrays["blk.0.attn_q.weight"].numpy(), ref["f16"])
    assert torch.equal(arrays["blk.0.attn_norm.weight"], ref["bf16"])
    for name, key in (("blk.0.attn_k.weight", "q4"), ("blk.0.attn_v.weight", "q6"), ("blk.0.ffn_down.weight", "iq2"),
                      ("blk.0.ffn_gate_exps.weight", "experts")):
        t = arrays[name]
        assert t.dtype == torch.uint8 and tuple(t.shape) == ref[key].shape, name
        assert np.array_equal(t.numpy(), ref[key]), name
        assert arrays[name[:-len(".weight")] + ".scales"].shape == (1,)
    # the wire rows dequantize like the oracle's (the bytes are the kernels' input)
    assert np.array_equal(okq.dequantize(arrays["blk.0.attn_v.weight"].numpy(), "q6_k"),
                          okq.dequantize(ref["q6"], "q6_k"))


def test_copy_and_zero_copy_agree(tmp_path):
    p, _ = _fixture(tmp_path, np.random.default_rng(2))
    a0, *_ = gguf.load_gguf(p, zero_copy=True)
    a1, *_ = gguf.load_gguf(p, zero_copy=False)
    for k in a0:
        assert torch.equal(a0[k], a1[k]), k
    # zero-copy views keep the mapping alive after the loader returns
    import gc
    gc.collect()
    assert torch.equal(a0["blk.0.attn_k.weight"], a1["blk.0.attn_k.weight"])


def test_alignment_honoured(tmp_path):
    p, ref = _fixture(tmp_path, np.random.default_rng(3), alignment=64)
    with gguf.GGUFFile(p) as g:
        assert g.alignment == 64 and g.data_offset % 64 == 0
        assert all(t.offset % 64 == 0 for t in g.tensors)
        i = [t.name for t in g.tensors].index("blk.0.attn_k.weight")
        assert np.array_equal(g.tensor(i, zero_copy=False).numpy(), ref["q4"])


def test_truncated_file_detected(tmp_path):
    p, _ = _fixture(tmp_path, np.random.default_rng(4))
    blob = open(p, "rb").read()
    cut = tmp_path / "cut.gguf"
    cut.write_bytes(blob[:-100])
    scan = gguf.scan_gguf(str(cut))
    assert scan.truncated and scan.expected_size == len(blob) and scan.size == len(blob) - 100
    with pytest.raises(gguf.GGUFError, match="truncated"):
        gguf.load_gguf(str(cut))
    # the metadata of a truncated file still reads
    assert gguf.scan_gguf(str(cut), include_tensors=False).kv["general.name"] == "scan-fixture"


@pytest.mark.parametrize("case", ["magic", "v1", "v4", "string_len", "tensor_type", "n_dims", "offset_align",
                                  "alignment_value", "partial_block", "short", "empty", "kv_type",
                                  "header_cut"])
def test_malformed_headers_raise(tmp_path, case):
    good_t = [("t", (256, 2), 12, bytes(288))]
    if case == "magic":
        blob = gguf_bytes(kv=BASIC_KV, magic=b"GGUX")
    elif case == "v1":
        blob = gguf_bytes(kv=BASIC_KV, version=1)
    elif case == "v4":
        blob = gguf_bytes(kv=BASIC_KV, version=4)
    elif case == "string_len":
        blob = bytearray(gguf_bytes(kv=[("k", STRING, "v")]))
        blob[24:32] = (2 ** 40).to_bytes(8, "little")          # the key's length
    elif case == "tensor_type":
        blob = gguf_bytes(tensors=[("t", (32,), 4, bytes(64))])  # type 4 is unassigned
    elif case == "n_dims":
        blob = gguf_bytes(tensors=[("t", (1, 1, 1, 1, 32), 0, bytes(128))])
    elif case == "offset_align":
        blob = bytearray(gguf_bytes(tensors=good_t))
        # tensor offset field: after magic/counts (24), the name (8 + 1), n_dims (4), dims (16), type (4)
        at = 24 + 9 + 4 + 16 + 4
        blob[at:at + 8] = (3).to_bytes(8, "little")
    elif case == "alignment_value":
        blob = gguf_bytes(kv=[("general.alignment", U32, 24)])
    elif case == "partial_block":
        blob = gguf_bytes(tensors=[("t", (300, 1), 12, bytes(144))])  # rows must hold whole blocks
    elif case == "short":
        blob = b"GGUF" + bytes(10)
    elif case == "empty":
        blob = b""
    elif case == "kv_type":
        blob = bytearray(gguf_bytes(kv=[("k", U8, 1)]))
        blob[24 + 9:24 + 13] = (13).to_bytes(4, "little")       # value type 13 does not exist
    else:  # header_cut: the tensor table runs past the end of the file
        blob = gguf_bytes(kv=BASIC_KV, tensors=good_t)[:60]
    p = tmp_path / "bad.gguf"
    p.write_bytes(bytes(blob))
    with pytest.raises(gguf.GGUFError):
        gguf.scan_gguf(str(p))


def test_missing_file_raises_oserror(tmp_path):
    with pytest.raises(OSError):
        gguf.scan_gguf(str(tmp_path / "absent.gguf"))


def test_type_table():
    from gmlx_amd import _lib
    L = _lib.lib()
    import ctypes
    b, n = ctypes.c_int32(), ctypes.c_int32()
    expect = {0: (1, 4), 1: (1, 2), 8: (32, 34), 12: (256, 144), 14: (256, 210), 16: (256, 66), 30: (1, 2),
              23: (256, 136), 39: (32, 17)}
    for t, bb in expect.items():
        assert L.kq_gguf_type_size(t, ctypes.byref(b), ctypes.byref(n)) == 0
        assert (b.value, n.value) == bb
    assert L.kq_gguf_type_size(4, None, None) == _lib.KQ_ERR_UNSUPPORTED_CODEC
    assert L.kq_gguf_type_size(1000, None, None) == _lib.KQ_ERR_UNSUPPORTED_CODEC
    # the three kernel codecs agree with the library's block sizes
    for t in (12, 14, 16):
        L.kq_gguf_type_size(t, ctypes.byref(b), ctypes.byref(n))
        assert n.value == L.kq_codec_block_bytes(t)


def test_split_shards(tmp_path):
    rng = np.random.default_rng(5)
    assert gguf.find_split_shards(str(tmp_path / "single.gguf")) == [str(tmp_path / "single.gguf")]
    q_a, q_b = _rng_wire(rng, "q4_k", 2, 256), _rng_wire(rng, "q6_k", 2, 256)
    s1 = write_gguf(tmp_path / "m-00001-of-00002.gguf", kv=BASIC_KV,
                    tensors=[("blk.0.attn_q.weight", (256, 2), 12, q_a.tobytes())])
    write_gguf(tmp_path / "m-00002-of-00002.gguf", kv=[("split.no", U16, 1)],
               tensors=[("blk.1.attn_q.weight", (256, 2), 14, q_b.tobytes())])
    shards = gguf.find_split_shards(s1)
    assert [s.rsplit("/", 1)[1] for s in shards] == ["m-00001-of-00002.gguf", "m-00002-of-00002.gguf"]
    arrays, codecs, arch, meta, shapes = gguf.load_gguf_wire_bytes(s1)
    assert arch == "llama" and "split.no" not in meta
    assert codecs == {"blk.0.attn_q.weight": "q4_k", "blk.1.attn_q.weight": "q6_k"}
    assert np.array_equal(arrays["blk.1.attn_q.weight"].numpy(), q_b)
    (tmp_path / "m-00002-of-00002.gguf").unlink()
    with pytest.raises(FileNotFoundError, match="1/2 shard"):
        gguf.find_split_shards(s1)


def test_qk_permutation_pinned():
    # llama.cpp's permute regroups each head's rows (0..D-1) as (2, D/2) -> (D/2, 2):
    # one head of D = 6 rows becomes 0 3 1 4 2 5
    rows = torch.arange(6).reshape(6, 1)
    fwd = gguf.qk_permute_wire_inverse(rows, 1)
    assert fwd.flatten().tolist() == [0, 3, 1, 4, 2, 5]
    assert gguf.qk_permute_wire(fwd, 1).flatten().tolist() == list(range(6))
    w = torch.randint(0, 255, (4 * 8, 144), dtype=torch.uint8)
    assert torch.equal(gguf.qk_permute_wire(gguf.qk_permute_wire_inverse(w, 4), 4), w)
    assert torch.equal(gguf.qk_permute_wire_inverse(gguf.qk_permute_wire(w, 4), 4), w)


def test_split_fused_gate_up():
    w = torch.arange(2 * 8 * 3, dtype=torch.int32).reshape(2, 8, 3).to(torch.uint8)
    g, u = gguf.split_fused_gate_up(w)
    assert torch.equal(g, w[:, :4]) and torch.equal(u, w[:, 4:])
    assert g.is_contiguous() and u.is_contiguous()
    with pytest.raises(ValueError):
        gguf.split_fused_gate_up(w[0])


def test_mutated_headers_parse_or_raise(tmp_path):
    """Random byte flips, overwrites and cuts of a valid file: every case
    parses or raises GGUFError; nothing reads outside the mapping (a stray
    read would crash this process)."""
    rng = np.random.default_rng(7)
    seed = gguf_bytes(kv=BASIC_KV, tensors=[("t0", (256, 2), 12, bytes(288)), ("t1", (64, 4), 0, bytes(1024))])
    p = tmp_path / "mut.gguf"
    opened = 0
    for _ in range(400):
        m = bytearray(seed)
        for _ in range(int(rng.integers(1, 6))):
            pos = int(rng.integers(0, len(m)))
            mode = int(rng.integers(0, 3))
            if mode == 0:
                m[pos] = int(rng.integers(0, 256))
            elif mode == 1 and pos + 8 <= len(m):
                m[pos:pos + 8] = int(rng.integers(0, 2 ** 63)).to_bytes(8, "little")
            else:
                del m[pos + 1:]
        p.write_bytes(bytes(m))
        try:
            s = gguf.scan_gguf(str(p), array_limit=64)
        except gguf.GGUFError:
            continue
        opened += 1
        assert s.size == len(m)
    assert opened > 0


def test_views_outlive_close(tmp_path):
    p, ref = _fixture(tmp_path, np.random.default_rng(8))
    with gguf.GGUFFile(p) as g:
        i = [t.name for t in g.tensors].index("blk.0.attn_k.weight")
        view = g.tensor(i)
    import gc
    del g
    gc.collect()
    assert np.array_equal(view.numpy(), ref["q4"])   # the mapping is still there
