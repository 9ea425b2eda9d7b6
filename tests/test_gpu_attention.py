"""Ragged GQA decode attention parity (kq_sdpa_decode_ragged through the C
ABI) against the fp64 per-row reference: the reference's construction is
per-row SDPA over each row's unpadded keys (tests/test_ragged_decode.py:48-58).
Pad poisoning must not leak (:126-148); outputs are deterministic."""
import numpy as np
import pytest

from helpers import BF16_TOL, TOL, attention_ref
from oracle import kquant as okq

pytestmark = pytest.mark.gpu


def _slabs(rng, lens, Hkv, D, dtype=np.float16):
    offs, ks, vs, off = [], [], [], 0
    for L in lens:
        ks.append(rng.normal(0, 1, size=(Hkv, L, D)).astype(dtype))
        vs.append(rng.normal(0, 1, size=(Hkv, L, D)).astype(dtype))
        offs.append(off)
        off += Hkv * L * D
    kflat = np.concatenate([k.reshape(-1) for k in ks] + [np.zeros(8, dtype)])
    vflat = np.concatenate([v.reshape(-1) for v in vs] + [np.zeros(8, dtype)])
    return offs, ks, vs, kflat, vflat


@pytest.mark.parametrize("D,Hq,Hkv", [(128, 32, 8), (64, 8, 8), (96, 12, 3), (256, 16, 1), (128, 16, 2)])
def test_ragged_slabs_fp16(D, Hq, Hkv):
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(D + Hq)
    lens = [1, 31, 33, 513, 1500, 0, 64]
    offs, ks, vs, kf, vf = _slabs(rng, lens, Hkv, D)
    q = rng.normal(0, 1, size=(len(lens), Hq, D)).astype(np.float16)
    scale = D ** -0.5
    out = ops.sdpa_decode_slabs(torch.from_numpy(q).cuda(), torch.from_numpy(kf).cuda(),
                                torch.from_numpy(vf).cuda(), offs, lens, Hkv, scale).float().cpu().numpy()
    ref = np.stack([attention_ref(q[b], ks[b], vs[b], scale) for b in range(len(lens))])
    assert okq.max_rel(out, ref) <= TOL, okq.max_rel(out, ref)
    assert np.all(out[5] == 0)          # empty row -> zeros (sum_exp == 0 branch of the reference)


def test_long_row_many_splits_and_determinism():
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(5)
    lens = [9000, 3, 4100]
    offs, ks, vs, kf, vf = _slabs(rng, lens, 2, 128)
    q = rng.normal(0, 1, size=(3, 8, 128)).astype(np.float16)
    args = (torch.from_numpy(q).cuda(), torch.from_numpy(kf).cuda(), torch.from_numpy(vf).cuda(), offs, lens, 2,
            128 ** -0.5)
    outs = [ops.sdpa_decode_slabs(*args).cpu().numpy() for _ in range(3)]
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint16), outs[0].view(np.uint16))
    ref = np.stack([attention_ref(q[b], ks[b], vs[b], 128 ** -0.5) for b in range(3)])
    assert okq.max_rel(outs[0].astype(np.float32), ref) <= TOL


def test_split_size_invariance(monkeypatch):
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(6)
    lens = [2000, 700]
    offs, ks, vs, kf, vf = _slabs(rng, lens, 4, 128)
    q = rng.normal(0, 1, size=(2, 16, 128)).astype(np.float16)
    ref = np.stack([attention_ref(q[b], ks[b], vs[b], 128 ** -0.5) for b in range(2)])
    for split in ("32", "96", "512", "1024", "4096"):
        monkeypatch.setenv("GMLX_KQ_SDPA_SPLIT", split)
        out = ops.sdpa_decode_slabs(torch.from_numpy(q).cuda(), torch.from_numpy(kf).cuda(),
                                    torch.from_numpy(vf).cuda(), offs, lens, 4, 128 ** -0.5)
        assert okq.max_rel(out.float().cpu().numpy(), ref) <= TOL, split


def _padded(rng, B, Hq, Hkv, L, D, dtype):
    import torch
    q = torch.from_numpy(rng.normal(0, 1, size=(B, Hq, 1, D)).astype(np.float32)).to(dtype)
    k = torch.from_numpy(rng.normal(0, 1, size=(B, Hkv, L, D)).astype(np.float32)).to(dtype)
    v = torch.from_numpy(rng.normal(0, 1, size=(B, Hkv, L, D)).astype(np.float32)).to(dtype)
    return q, k, v


@pytest.mark.parametrize("dtype_name", ["float16", "bfloat16"])
def test_reference_layout_with_pads(dtype_name):
    """ragged_decode_attention(q, k, v, pads, scale) on [B, Hkv, L, D]."""
    import torch
    from gmlx_amd import ops
    dtype = getattr(torch, dtype_name)
    rng = np.random.default_rng(21)
    B, Hq, Hkv, L, D = 3, 16, 2, 4096, 256
    pads = [0, 1000, 2000]
    q, k, v = _padded(rng, B, Hq, Hkv, L, D, dtype)
    got = ops.ragged_decode_attention(q.cuda(), k.cuda(), v.cuda(), pads, D ** -0.5)
    assert got is not None and got.shape == (B, Hq, 1, D)
    qf, kf, vf = q.float().numpy(), k.float().numpy(), v.float().numpy()
    ref = np.stack([attention_ref(qf[b, :, 0], kf[b, :, pads[b]:], vf[b, :, pads[b]:], D ** -0.5)
                    for b in range(B)])
    tol = TOL if dtype == torch.float16 else BF16_TOL
    assert okq.max_rel(got.float().cpu().numpy()[:, :, 0], ref) <= tol


def test_pads_are_honored():
    """Poisoning the pad region cannot change the output (bit-exact)."""
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(1)
    B, Hq, Hkv, L, D = 2, 16, 2, 4096, 128
    pads = [512, 0]
    q, k, v = _padded(rng, B, Hq, Hkv, L, D, torch.bfloat16)
    clean = ops.ragged_decode_attention(q.cuda(), k.cuda(), v.cuda(), pads, D ** -0.5)
    k2 = k.clone()
    k2[0, :, :pads[0]] = 40.0
    v2 = v.clone()
    v2[0, :, :pads[0]] = -40.0
    dirty = ops.ragged_decode_attention(q.cuda(), k2.cuda(), v2.cuda(), pads, D ** -0.5)
    assert torch.equal(clean.cpu(), dirty.cpu())


@pytest.mark.parametrize("starts_kind", ["device", "host", "cpu_tensor", "none"])
def test_sdpa_decode_gqa_starts(starts_kind):
    """kq.sdpa_decode_gqa(starts=) (gmlx/gemma4_batched_sdpa.py:210-226)
    against the fp64 per-row reference over keys [starts[b], L)."""
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(3)
    B, Hq, Hkv, L, D = 4, 8, 1, 640, 64
    q, k, v = _padded(rng, B, Hq, Hkv, L, D, torch.float16)
    st = [0, 100, 639, 7] if starts_kind != "none" else [0] * B
    arg = {"device": torch.tensor(st, dtype=torch.int32).cuda(), "host": st,
           "cpu_tensor": torch.tensor(st, dtype=torch.int64), "none": None}[starts_kind]
    got = ops.sdpa_decode_gqa(q.cuda(), k.cuda(), v.cuda(), 0.125, starts=arg)
    qf, kf, vf = q.float().numpy(), k.float().numpy(), v.float().numpy()
    ref = np.stack([attention_ref(qf[b, :, 0], kf[b, :, st[b]:], vf[b, :, st[b]:], 0.125) for b in range(B)])
    assert okq.max_rel(got.float().cpu().numpy()[:, :, 0], ref) <= TOL


def test_decode_steps_sync_free_and_table_free():
    """A decode loop (keys L, L + 1, L + 2 with the same pads / device starts)
    makes no host synchronisation and builds no new device tables: the
    reference passes device starts for exactly this (gmlx/quantized_sdpa_fix.py:
    37-45, 88-93) and memoises pads per batch (gmlx/cascade_sdpa.py:79-105)."""
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(8)
    B, Hq, Hkv, Lmax, D = 3, 16, 4, 2100, 128
    q, k, v = _padded(rng, B, Hq, Hkv, Lmax, D, torch.float16)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    pads = [5, 0, 1024]
    dev_starts = torch.tensor(pads, dtype=torch.int32, device="cuda")
    ops.ragged_decode_attention(qd, kd[:, :, :2000], vd[:, :, :2000], pads, D ** -0.5)  # first sight of the pads
    torch.cuda.synchronize()
    n_tables = len(ops._STARTS)
    outs = []
    torch.cuda.set_sync_debug_mode("error")
    try:
        for L in (2001, 2002, 2003):
            outs.append(ops.ragged_decode_attention(qd, kd[:, :, :L], vd[:, :, :L], pads, D ** -0.5))
            outs.append(ops.sdpa_decode_gqa(qd, kd[:, :, :L], vd[:, :, :L], D ** -0.5, starts=dev_starts))
    finally:
        torch.cuda.set_sync_debug_mode(0)
    assert len(ops._STARTS) == n_tables
    qf, kf, vf = q.float().numpy(), k.float().numpy(), v.float().numpy()
    for i, L in enumerate((2001, 2002, 2003)):
        ref = np.stack([attention_ref(qf[b, :, 0], kf[b, :, pads[b]:L], vf[b, :, pads[b]:L], D ** -0.5)
                        for b in range(B)])
        for o in outs[2 * i:2 * i + 2]:
            assert okq.max_rel(o.float().cpu().numpy()[:, :, 0], ref) <= TOL


@pytest.mark.parametrize("D,Hq,Hkv,dtype_name", [(128, 32, 8, "float16"), (64, 8, 8, "float16"),
                                                 (256, 16, 2, "float16"), (128, 16, 4, "bfloat16")])
def test_sdpa_decode_gqa_q8_kv(D, Hq, Hkv, dtype_name):
    """Quantized-KV form of sdpa_decode_gqa (gmlx/quantized_sdpa_fix.py:170-182):
    an 8-bit affine cache (bits 8, group 64, mlx's uint32 wire) against fp64
    attention over the dequantized keys and values, ragged starts included."""
    import torch
    from gmlx_amd import ops
    from helpers import q8_affine
    rng = np.random.default_rng(D + Hq)
    B, L = 5, 1300
    kf = rng.normal(0, 1, size=(B, Hkv, L, D)).astype(np.float32)
    vf = rng.normal(0, 1, size=(B, Hkv, L, D)).astype(np.float32)
    kw, ks, kb, kd = q8_affine(kf, dtype_name)
    vw, vs, vb, vd = q8_affine(vf, dtype_name)
    tdt = getattr(torch, dtype_name)
    q = torch.from_numpy(rng.normal(0, 1, size=(B, Hq, 1, D)).astype(np.float32)).to(tdt)
    starts = [0, 17, 600, 1299, 3]
    scale = D ** -0.5
    out = ops.sdpa_decode_gqa(q.cuda(), kw.cuda(), vw.cuda(), scale, starts=starts, k_scales=ks.cuda(),
                              k_biases=kb.cuda(), v_scales=vs.cuda(), v_biases=vb.cuda())
    assert out.dtype == tdt and tuple(out.shape) == (B, Hq, 1, D)
    qd = q.double().numpy()[:, :, 0]
    ref = np.stack([attention_ref(qd[b], kd[b][:, starts[b]:], vd[b][:, starts[b]:], scale) for b in range(B)])
    tol = BF16_TOL if dtype_name == "bfloat16" else TOL
    assert okq.max_rel(out.float().cpu().numpy()[:, :, 0], ref) <= tol


@pytest.mark.parametrize("B,Hq,Hkv,dtype_name", [(2, 16, 1, "float16"), (16, 8, 2, "float16"),
                                                 (5, 32, 4, "bfloat16"), (16, 16, 16, "bfloat16")])
def test_head_dim_512(B, Hq, Hkv, dtype_name):
    """Head dim 512, the only one the reference's batched starts= route claims
    (gmlx/gemma4_batched_sdpa.py:172-177), at B 2..16 and G 1..16: the
    16-bit and the 8-bit affine KV forms of sdpa_decode_gqa against the fp64
    per-row reference over keys [starts[b], L) (a 16-token tile per step at
    this head dim)."""
    import torch
    from gmlx_amd import ops
    from helpers import q8_affine
    rng = np.random.default_rng(B * 7 + Hq)
    D, L = 512, 900
    tdt = getattr(torch, dtype_name)
    tol = BF16_TOL if dtype_name == "bfloat16" else TOL
    kf = rng.normal(0, 1, size=(B, Hkv, L, D)).astype(np.float32)
    vf = rng.normal(0, 1, size=(B, Hkv, L, D)).astype(np.float32)
    q = torch.from_numpy(rng.normal(0, 1, size=(B, Hq, 1, D)).astype(np.float32)).to(tdt)
    starts = rng.integers(0, L - 1, size=B).tolist()
    starts[0] = 0
    scale = D ** -0.5
    dev_st = torch.tensor(starts, dtype=torch.int32, device="cuda")
    print(f"hd512 B={B} Hq={Hq} Hkv={Hkv} {dtype_name}", flush=True)
    k16, v16 = torch.from_numpy(kf).to(tdt), torch.from_numpy(vf).to(tdt)
    out = ops.sdpa_decode_gqa(q.cuda(), k16.cuda(), v16.cuda(), scale, starts=dev_st)
    qd = q.double().numpy()[:, :, 0]
    kd16, vd16 = k16.double().numpy(), v16.double().numpy()
    ref = np.stack([attention_ref(qd[b], kd16[b][:, starts[b]:], vd16[b][:, starts[b]:], scale) for b in range(B)])
    assert okq.max_rel(out.float().cpu().numpy()[:, :, 0], ref) <= tol
    kw, ks, kb, kd = q8_affine(kf, dtype_name)
    vw, vs, vb, vd = q8_affine(vf, dtype_name)
    out8 = ops.sdpa_decode_gqa(q.cuda(), kw.cuda(), vw.cuda(), scale, starts=dev_st, k_scales=ks.cuda(),
                               k_biases=kb.cuda(), v_scales=vs.cuda(), v_biases=vb.cuda())
    ref8 = np.stack([attention_ref(qd[b], kd[b][:, starts[b]:], vd[b][:, starts[b]:], scale) for b in range(B)])
    assert okq.max_rel(out8.float().cpu().numpy()[:, :, 0], ref8) <= tol
    # the ragged route keeps the reference's head dims and declines 512
    assert ops.ragged_decode_attention(q.cuda(), k16.cuda(), v16.cuda(), starts, scale) is None


@pytest.mark.parametrize("split", [None, "512", "1024"])
@pytest.mark.parametrize("dtype_name", ["float16", "bfloat16"])
def test_batch_row_equals_single_row(split, dtype_name, monkeypatch):
    """Row b of a batched call is bitwise the same call made on row b alone:
    the reference's same-bucket property (tests/test_ragged_decode.py:94-114,
    one plan for the batch and for each row, no drift at all).  Covered:
    ragged_decode_attention on [B, Hkv, L, D] with the reference's live pads
    (:97), sdpa_decode_gqa with device starts over the 16-bit and the 8-bit
    affine cache, and the per-row slab layout.  Splits run 512 or 1024 tokens
    by the launch's size, so the batched and the single-row call are also
    compared with the split forced either way."""
    import torch
    from gmlx_amd import ops
    from helpers import q8_affine
    if split is not None:
        monkeypatch.setenv("GMLX_KQ_SDPA_SPLIT", split)
    tdt = getattr(torch, dtype_name)
    rng = np.random.default_rng(94)
    B, Hq, Hkv, L, D = 3, 32, 8, 14772, 128
    pads = [248, 217, 0]
    q, k, v = _padded(rng, B, Hq, Hkv, L, D, tdt)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    print(f"batch-row ragged split={split} {dtype_name}", flush=True)
    full = ops.ragged_decode_attention(qd, kd, vd, pads, D ** -0.5)
    assert full is not None
    for b in range(B):
        one = ops.ragged_decode_attention(qd[b:b + 1], kd[b:b + 1], vd[b:b + 1], pads[b:b + 1], D ** -0.5)
        assert torch.equal(one[0], full[b]), ("ragged", b)
    starts = torch.tensor(pads, dtype=torch.int32, device="cuda")
    full = ops.sdpa_decode_gqa(qd, kd, vd, D ** -0.5, starts=starts)
    for b in range(B):
        one = ops.sdpa_decode_gqa(qd[b:b + 1], kd[b:b + 1], vd[b:b + 1], D ** -0.5, starts=starts[b:b + 1])
        assert torch.equal(one[0], full[b]), ("starts", b)
    Lq = 3000  # the 8-bit affine cache
    kw, ks, kb, _ = q8_affine(k[:, :, :Lq].float().numpy(), dtype_name)
    vw, vs, vb, _ = q8_affine(v[:, :, :Lq].float().numpy(), dtype_name)
    kw, ks, kb, vw, vs, vb = (t.cuda() for t in (kw, ks, kb, vw, vs, vb))
    full = ops.sdpa_decode_gqa(qd, kw, vw, D ** -0.5, starts=starts, k_scales=ks, k_biases=kb,
                               v_scales=vs, v_biases=vb)
    for b in range(B):
        sl = slice(b, b + 1)
        one = ops.sdpa_decode_gqa(qd[sl], kw[sl], vw[sl], D ** -0.5, starts=starts[sl], k_scales=ks[sl],
                                  k_biases=kb[sl], v_scales=vs[sl], v_biases=vb[sl])
        assert torch.equal(one[0], full[b]), ("q8", b)
    if dtype_name == "float16":
        lens = [1, 700, 2500, 0, 1333]
        offs, ks_, vs_, kf, vf = _slabs(rng, lens, Hkv, D)
        qs = torch.from_numpy(rng.normal(0, 1, size=(len(lens), Hq, D)).astype(np.float16)).cuda()
        kf, vf = torch.from_numpy(kf).cuda(), torch.from_numpy(vf).cuda()
        full = ops.sdpa_decode_slabs(qs, kf, vf, offs, lens, Hkv, D ** -0.5)
        for b in range(len(lens)):
            one = ops.sdpa_decode_slabs(qs[b:b + 1], kf, vf, offs[b:b + 1], lens[b:b + 1], Hkv, D ** -0.5)
            assert torch.equal(one[0], full[b]), ("slabs", b)
