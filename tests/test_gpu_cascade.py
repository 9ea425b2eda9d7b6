"""Cascade shared-prefix decode attention (kq_sdpa_decode_gqa_cascade through
the C ABI) against the fp64 masked reference.

Construction follows the reference's tests (tests/test_cascade_sdpa.py:66-93,
:155-197): a [B, Hkv, maxpad + P + sp, D] cache whose rows each hold one copy
of a shared P-token prefix at [pads[b], pads[b] + P) and private tokens after
it; the op is called the way the claim slices it (gmlx/cascade_sdpa.py:
95-105, 211-248): k_shared = keys[0:1, :, pads[0]:pads[0] + P], private
slab = keys[:, :, c0:] with c0 = min_b(pads[b] + P) and
starts[b] = pads[b] + P - c0.  The reference result is attention over each
row's keys [pads[b], L - qL + i] of the whole buffer (left padding plus the
end-aligned causal of a verify block, :108-117)."""
import numpy as np
import pytest

from helpers import BF16_TOL, TOL, attention_ref
from oracle import kquant as okq

pytestmark = pytest.mark.gpu


def _shared_batch(rng, B, Hkv, P, sp, pads, D, dtype):
    L = max(pads) + P + sp
    kb = rng.normal(0, 1, size=(B, Hkv, L, D)).astype(np.float32)
    vb = rng.normal(0, 1, size=(B, Hkv, L, D)).astype(np.float32)
    for b in range(1, B):  # every row carries row 0's prefix copy
        kb[b, :, pads[b]:pads[b] + P] = kb[0, :, pads[0]:pads[0] + P]
        vb[b, :, pads[b]:pads[b] + P] = vb[0, :, pads[0]:pads[0] + P]
    return kb, vb, L


def _masked_ref(q, kb, vb, pads, scale):
    """fp64: q (B, Hq, qL, D); row (b, i) sees keys [pads[b], L - qL + i]."""
    B, Hq, qL, D = q.shape
    L = kb.shape[2]
    out = np.zeros((B, Hq, qL, D), np.float64)
    for b in range(B):
        for i in range(qL):
            end = L - qL + i + 1
            out[b, :, i] = attention_ref(q[b, :, i], kb[b, :, pads[b]:end], vb[b, :, pads[b]:end], scale)
    return out


def _cascade(torch, ops, q, kb, vb, pads, P, scale, starts_on_device=True):
    """Slice the buffer the way the reference's claim does and call the op."""
    c0 = min(p + P for p in pads)
    starts = [p + P - c0 for p in pads]
    l0 = pads[0]
    st = torch.tensor(starts, dtype=torch.int32, device="cuda") if starts_on_device else starts
    return ops.sdpa_decode_gqa_cascade(q, kb[0:1, :, l0:l0 + P], vb[0:1, :, l0:l0 + P], kb[:, :, c0:],
                                       vb[:, :, c0:], scale, starts=st)


def _run(B, Hq, Hkv, D, P, sp, pads, qL, dtype_name, seed=0, starts_on_device=True):
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(seed)
    kb, vb, L = _shared_batch(rng, B, Hkv, P, sp, pads, D, np.float32)
    q = rng.normal(0, 1, size=(B, Hq, qL, D)).astype(np.float32)
    tdt = getattr(torch, dtype_name)
    kt, vt, qt = (torch.from_numpy(a).to(tdt).cuda() for a in (kb, vb, q))
    scale = D ** -0.5
    print(f"cascade B={B} Hq={Hq} Hkv={Hkv} D={D} P={P} sp={sp} pads={pads} qL={qL} {dtype_name}", flush=True)
    out = _cascade(torch, ops, qt, kt, vt, pads, P, scale, starts_on_device)
    torch.cuda.synchronize()
    # the reference sees the inputs as rounded to the kernel's dtype
    ref = _masked_ref(qt.float().cpu().numpy(), kt.float().cpu().numpy(), vt.float().cpu().numpy(), pads, scale)
    return out, ref


@pytest.mark.parametrize("pads", [[0, 0, 0, 0], [0, 64, 128, 32]])
def test_decode_width_matches_masked_reference(pads):
    out, ref = _run(4, 16, 8, 128, 1024, 96, pads, 1, "float16")
    assert okq.max_rel(out.float().cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("qL,pads", [(4, [0, 0, 0]), (8, [0, 64, 32]), (2, [5, 0, 17, 3])])
def test_verify_width_matches_masked_reference(qL, pads):
    out, ref = _run(len(pads), 16, 8, 128, 1024, 96, pads, qL, "float16", seed=qL)
    assert okq.max_rel(out.float().cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("D,Hq,Hkv", [(64, 8, 8), (96, 12, 3), (256, 16, 1), (128, 32, 8), (128, 48, 4)])
def test_head_shapes(D, Hq, Hkv):
    # G = 1, 4, 16, 4, 12: 16, 4, 1, 4 and 1 rows per prefix tile load
    out, ref = _run(5, Hq, Hkv, D, 700, 40, [3, 0, 9, 0, 1], 3, "float16", seed=D)
    assert okq.max_rel(out.float().cpu().numpy(), ref) <= TOL


def test_bfloat16_host_starts():
    out, ref = _run(3, 16, 4, 128, 1500, 300, [0, 7, 2], 1, "bfloat16", starts_on_device=False)
    assert okq.max_rel(out.float().cpu().numpy(), ref) <= BF16_TOL


def test_long_prefix_many_splits_and_determinism():
    """P spans many splits (prefix units of 16/G rows) and the private tails
    several; repeated calls are bitwise equal."""
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(9)
    pads, P, sp, qL = [0, 300, 40, 7, 0, 1000, 2, 64], 9000, 1200, 2
    kb, vb, L = _shared_batch(rng, 8, 8, P, sp, pads, 128, np.float32)
    q = rng.normal(0, 1, size=(8, 32, qL, 128)).astype(np.float32)
    kt, vt, qt = (torch.from_numpy(a).half().cuda() for a in (kb, vb, q))
    outs = [_cascade(torch, ops, qt, kt, vt, pads, P, 128 ** -0.5).cpu().numpy() for _ in range(3)]
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint16), outs[0].view(np.uint16))
    ref = _masked_ref(qt.float().cpu().numpy(), kt.float().cpu().numpy(), vt.float().cpu().numpy(), pads,
                      128 ** -0.5)
    assert okq.max_rel(outs[0].astype(np.float32), ref) <= TOL


def test_agrees_with_ragged_route_on_the_buffer():
    """Decode width: the cascade over the sliced buffer and the ragged kernel
    over the whole left-padded buffer compute the same attention."""
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(3)
    pads, P = [0, 64, 128, 32, 5, 0], 2048
    kb, vb, L = _shared_batch(rng, 6, 8, P, 200, pads, 128, np.float32)
    q = rng.normal(0, 1, size=(6, 32, 1, 128)).astype(np.float32)
    kt, vt, qt = (torch.from_numpy(a).half().cuda() for a in (kb, vb, q))
    casc = _cascade(torch, ops, qt, kt, vt, pads, P, 128 ** -0.5).float().cpu().numpy()
    rag = ops.ragged_decode_attention(qt, kt, vt, pads, 128 ** -0.5).float().cpu().numpy()
    assert okq.max_rel(casc, rag.astype(np.float64)) <= TOL


def test_split_size_invariance(monkeypatch):
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(4)
    pads, P = [0, 3, 70], 1100
    kb, vb, L = _shared_batch(rng, 3, 2, P, 90, pads, 128, np.float32)
    q = rng.normal(0, 1, size=(3, 8, 3, 128)).astype(np.float32)
    kt, vt, qt = (torch.from_numpy(a).half().cuda() for a in (kb, vb, q))
    ref = _masked_ref(qt.float().cpu().numpy(), kt.float().cpu().numpy(), vt.float().cpu().numpy(), pads,
                      128 ** -0.5)
    for split, split1 in (("32", "0"), ("96", "64"), ("512", "0"), ("512", "1100"), ("4096", "2048")):
        monkeypatch.setenv("GMLX_KQ_SDPA_SPLIT", split)
        monkeypatch.setenv("GMLX_KQ_CASCADE_SPLIT", split1)
        out = _cascade(torch, ops, qt, kt, vt, pads, P, 128 ** -0.5).float().cpu().numpy()
        assert okq.max_rel(out, ref) <= TOL, (split, split1)


def test_rejects_bad_shapes():
    import torch
    from gmlx_amd import ops
    q = torch.zeros(2, 8, 1, 128, dtype=torch.float16, device="cuda")
    ks = torch.zeros(1, 2, 64, 128, dtype=torch.float16, device="cuda")
    kp = torch.zeros(2, 2, 16, 128, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        ops.sdpa_decode_gqa_cascade(q, ks, ks, kp[:1], kp[:1], 0.1)         # batch mismatch
    with pytest.raises(ValueError):
        ops.sdpa_decode_gqa_cascade(q[..., :80], ks[..., :80], ks[..., :80], kp[..., :80], kp[..., :80], 0.1)
    with pytest.raises(ValueError):   # the quantized form needs all eight scale / bias tensors
        ops.sdpa_decode_gqa_cascade(q, ks, ks, kp, kp, 0.1, k_shared_scales=ks)
    with pytest.raises(TypeError):
        ops.sdpa_decode_gqa_cascade(q, ks, ks, kp, kp, 0.1, k_scales=ks)


# ------------------------------------------------ through the host route

class _StampedCache:
    def __init__(self, pads, P=None):
        import torch
        self.left_padding = torch.tensor(pads)
        self._right_padding = None
        if P is not None:
            self._gmlx_cascade = {"P": P, "tok": ()}


def _route_case(B, qL, pads, P=1024, sp=96, seed=21):
    import torch
    rng = np.random.default_rng(seed)
    kb, vb, L = _shared_batch(rng, B, 8, P, sp, pads, 128, np.float32)
    q = rng.normal(0, 1, size=(B, 16, qL, 128)).astype(np.float32)
    kt, vt, qt = (torch.from_numpy(a).half().cuda() for a in (kb, vb, q))
    ref = _masked_ref(qt.float().cpu().numpy(), kt.float().cpu().numpy(), vt.float().cpu().numpy(), pads, 0.125)
    return qt, kt, vt, ref


@pytest.mark.parametrize("qL,mask,pads", [(1, None, [0, 64, 128, 32]), (4, "causal", [0, 64, 32]),
                                           (8, "causal", [0, 0, 0])])
def test_route_claims_stamped_calls(qL, mask, pads):
    from gmlx_amd import decode_route as dr

    def stock(*a, **k):
        raise AssertionError("a claimable stamped call fell through")

    qt, kt, vt, ref = _route_case(len(pads), qL, pads)
    route = dr.make_route(stock)
    n0 = dr.claims()
    out = route(qt, kt, vt, cache=_StampedCache(pads, P=1024), scale=0.125, mask=mask)
    assert dr.claims() == n0 + 1
    assert okq.max_rel(out.float().cpu().numpy(), ref) <= TOL


def test_left_padded_route_order():
    """Stamped batch: the cascade claims; unstamped: the ragged kernel runs.
    Both agree with the masked reference."""
    from gmlx_amd import decode_route as dr
    pads = [0, 64, 128, 32]
    qt, kt, vt, ref = _route_case(4, 1, pads)
    n0 = dr.claims()
    casc = dr.left_padded_attention(qt, kt, vt, cache=_StampedCache(pads, P=1024), scale=0.125)
    assert dr.claims() == n0 + 1
    rag = dr.left_padded_attention(qt, kt, vt, cache=_StampedCache(pads), scale=0.125)
    assert dr.claims() == n0 + 1
    for out in (casc, rag):
        assert okq.max_rel(out.float().cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("qL,pads,dtype_name", [(1, [0, 64, 128, 32], "float16"), (4, [0, 64, 32], "float16"),
                                                (1, [5, 0, 9], "bfloat16"), (4, [5, 0, 9], "bfloat16")])
def test_quantized_kv_cascade(qL, pads, dtype_name):
    """The 8-bit affine KV form (gmlx/cascade_sdpa.py:216-236): wire, scales
    and biases sliced from one quantized buffer the way the claim slices
    them; against the masked fp64 reference over the dequantized buffer.
    qL = 4 gives 12 query rows at G = 2: two row blocks per prefix wave (the
    bf16 form of which keeps chunk-sized K loads)."""
    import torch
    from gmlx_amd import ops
    from helpers import q8_affine
    rng = np.random.default_rng(qL + len(pads))
    B, Hkv, Hq, D, P, sp = len(pads), 8, 16, 128, 1024, 96
    kb_, vb_, L = _shared_batch(rng, B, Hkv, P, sp, pads, D, np.float32)
    kw, ks, kbias, kd = q8_affine(kb_, dtype_name)
    vw, vs, vbias, vd = q8_affine(vb_, dtype_name)
    for b in range(1, B):   # the prefix copies must stay identical after quantization
        assert np.array_equal(kd[b, :, pads[b]:pads[b] + P], kd[0, :, pads[0]:pads[0] + P])
    tdt = getattr(torch, dtype_name)
    q = torch.from_numpy(rng.normal(0, 1, size=(B, Hq, qL, D)).astype(np.float32)).to(tdt)
    c0 = min(pads) + P
    starts = torch.tensor([p + P - c0 for p in pads], dtype=torch.int32, device="cuda")
    l0 = pads[0]
    kw, ks, kbias, vw, vs, vbias = (t.cuda() for t in (kw, ks, kbias, vw, vs, vbias))
    sl = lambda t: t[0:1, :, l0:l0 + P]  # noqa: E731
    pr = lambda t: t[:, :, c0:]  # noqa: E731
    out = ops.sdpa_decode_gqa_cascade(
        q.cuda(), sl(kw), sl(vw), pr(kw), pr(vw), 0.125, starts=starts,
        k_shared_scales=sl(ks), k_shared_biases=sl(kbias), v_shared_scales=sl(vs), v_shared_biases=sl(vbias),
        k_priv_scales=pr(ks), k_priv_biases=pr(kbias), v_priv_scales=pr(vs), v_priv_biases=pr(vbias))
    ref = _masked_ref(q.double().numpy(), kd, vd, pads, 0.125)
    tol = BF16_TOL if dtype_name == "bfloat16" else TOL
    assert okq.max_rel(out.float().cpu().numpy(), ref) <= tol


def test_route_claims_quantized_cache():
    """An 8-bit group-64 cache's (wire, scales, biases) K / V go through the
    claim into the quantized cascade (gmlx/cascade_sdpa.py:146-162)."""
    import torch
    from gmlx_amd import decode_route as dr
    from helpers import q8_affine
    rng = np.random.default_rng(31)
    pads, P, sp = [0, 64, 128, 32], 1024, 96
    kb_, vb_, L = _shared_batch(rng, 4, 8, P, sp, pads, 128, np.float32)
    kw, ks, kbias, kd = q8_affine(kb_)
    vw, vs, vbias, vd = q8_affine(vb_)
    q = torch.from_numpy(rng.normal(0, 1, size=(4, 16, 1, 128)).astype(np.float32)).half()
    cache = _StampedCache(pads, P=1024)
    cache.bits, cache.group_size = 8, 64
    n0 = dr.claims()
    out = dr.cascade_claim(q.cuda(), (kw.cuda(), ks.cuda(), kbias.cuda()), (vw.cuda(), vs.cuda(), vbias.cuda()),
                           cache, 0.125)
    assert out is not None and dr.claims() == n0 + 1
    ref = _masked_ref(q.double().numpy(), kd, vd, pads, 0.125)
    assert okq.max_rel(out.float().cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("B,Hq,Hkv,qL,dtype_name", [(8, 8, 2, 1, "float16"), (4, 16, 4, 2, "float16"),
                                                    (2, 16, 1, 1, "bfloat16")])
def test_head_dim_512(B, Hq, Hkv, qL, dtype_name):
    """Head dim 512 inside the claim's width gate for it (B * G * qL <= 32,
    gmlx/cascade_sdpa.py:66, 194): 16-bit KV against the masked fp64
    reference."""
    pads = [3 * b % 11 for b in range(B)]
    out, ref = _run(B, Hq, Hkv, 512, 1100, 70, pads, qL, dtype_name, seed=B + qL)
    tol = BF16_TOL if dtype_name == "bfloat16" else TOL
    assert okq.max_rel(out.float().cpu().numpy(), ref) <= tol


def test_quantized_kv_cascade_head_dim_512():
    """The 8-bit affine KV cascade at head dim 512 (whole 64-value groups)."""
    import torch
    from gmlx_amd import ops
    from helpers import q8_affine
    rng = np.random.default_rng(512)
    pads = [0, 40, 12, 7]
    B, Hkv, Hq, D, P, sp, qL = len(pads), 2, 8, 512, 1024, 80, 1
    kb_, vb_, L = _shared_batch(rng, B, Hkv, P, sp, pads, D, np.float32)
    kw, ks, kbias, kd = q8_affine(kb_, "float16")
    vw, vs, vbias, vd = q8_affine(vb_, "float16")
    q = torch.from_numpy(rng.normal(0, 1, size=(B, Hq, qL, D)).astype(np.float32)).half()
    c0 = min(pads) + P
    starts = torch.tensor([p + P - c0 for p in pads], dtype=torch.int32, device="cuda")
    l0 = pads[0]
    kw, ks, kbias, vw, vs, vbias = (t.cuda() for t in (kw, ks, kbias, vw, vs, vbias))
    sl = lambda t: t[0:1, :, l0:l0 + P]  # noqa: E731
    pr = lambda t: t[:, :, c0:]  # noqa: E731
    out = ops.sdpa_decode_gqa_cascade(
        q.cuda(), sl(kw), sl(vw), pr(kw), pr(vw), D ** -0.5, starts=starts,
        k_shared_scales=sl(ks), k_shared_biases=sl(kbias), v_shared_scales=sl(vs), v_shared_biases=sl(vbias),
        k_priv_scales=pr(ks), k_priv_biases=pr(kbias), v_priv_scales=pr(vs), v_priv_biases=pr(vbias))
    ref = _masked_ref(q.double().numpy(), kd, vd, pads, D ** -0.5)
    assert okq.max_rel(out.float().cpu().numpy(), ref) <= TOL
