"""MoE expert-gather family parity through the C ABI: routing, gather_qmm
(KQuantSwitchLinear, tests/test_native_fp.py:420-428 convention), the fused
GLU gather, the per-pair down gather, the routing mix (fp32, slots in order),
and the router top-k (gmlx/modules.py:754-760 stock form)."""
import numpy as np
import pytest

from helpers import TOL, fp16_rows, quantized_weights
from oracle import kquant as okq

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _experts(rng, codec, E, N, K):
    if codec == "iq2_xxs":
        return okq.random_valid_blocks(rng, codec, E * N * K // 256).reshape(E, N, -1)
    return np.stack([quantized_weights(rng, codec, N, K) for _ in range(E)])


@pytest.mark.parametrize("E,T,k", [(16, 37, 4), (128, 32, 8), (2000, 300, 8), (4096, 1250, 8), (256, 1, 8),
                                   (4, 64, 4), (1024, 8, 8), (60, 64, 6), (128, 512, 8), (3, 700, 2)])
def test_route_groups_pairs_stably(E, T, k):
    """Stable counting sort by expert: segment list, starts and pair order
    (per-chunk ranks with the chunk histograms in LDS; more experts than
    threads; histograms past LDS, the ballot-per-expert form; heavy
    duplication inside a 64-pair chunk; out-of-range ids)."""
    from gmlx_amd import ops
    rng = np.random.default_rng(E + T)
    idx = rng.integers(0, E, size=(T, k)).astype(np.int32)
    if T > 1:
        idx[0, 0], idx[-1, -1] = -1, E + 5  # never routed
    seg, order = ops.moe_route(_dev(idx), E)
    seg, order = seg.cpu().numpy(), order.cpu().numpy()
    flat = idx.reshape(-1)
    P = flat.size
    valid = (flat >= 0) & (flat < E)
    S = seg[0]
    uniq = np.unique(flat[valid])
    assert S == len(uniq)
    assert list(seg[1:1 + S]) == list(uniq)
    counts = np.array([(flat == e).sum() for e in uniq])
    starts = np.concatenate([[0], np.cumsum(counts)])
    assert list(seg[1 + E:1 + E + S + 1]) == list(starts)
    want = np.argsort(np.where(valid, flat, E + 10), kind="stable")[:valid.sum()]
    assert np.array_equal(order[:valid.sum()], want)
    assert np.array_equal(order[P:2 * P], np.where(valid, flat, -1))


@pytest.mark.parametrize("codec", ["q4_k", "q6_k", "iq2_xxs"])
def test_gather_qmm(codec):
    from gmlx_amd import ops
    rng = np.random.default_rng(1)
    E, N, K, T, k = 12, 80, 512, 9, 3
    w = _experts(rng, codec, E, N, K)
    deq = okq.dequantize(w, codec).astype(np.float64)
    x = fp16_rows(rng, T, K)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    got = ops.gather_qmm(_dev(x).reshape(T, 1, 1, K), _dev(w), None, codec, indices=_dev(idx))
    assert tuple(got.shape) == (T, k, 1, N)
    ref = np.stack([[deq[idx[t, s]] @ x[t].astype(np.float64) for s in range(k)] for t in range(T)])
    assert okq.max_rel(got.float().cpu().numpy()[:, :, 0], ref) <= TOL


def test_gather_many_rows_per_expert():
    """Segments larger than one 64-row chunk (prefill-sized)."""
    from gmlx_amd import ops
    rng = np.random.default_rng(2)
    E, N, K, T, k = 3, 48, 256, 150, 2
    w = _experts(rng, "q4_k", E, N, K)
    deq = okq.dequantize(w, "q4_k").astype(np.float64)
    x = fp16_rows(rng, T, K)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    got = ops.gather_qmm(_dev(x), _dev(w), None, "q4_k", indices=_dev(idx)).float().cpu().numpy()[:, :, 0]
    ref = np.stack([[deq[idx[t, s]] @ x[t].astype(np.float64) for s in range(k)] for t in range(T)])
    assert okq.max_rel(got, ref) <= TOL


@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_moe_glu_then_down_then_mix(act):
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(3)
    E, D, I, T, k = 16, 512, 256, 5, 4
    gw = _experts(rng, "q4_k", E, I, D)
    uw = _experts(rng, "q4_k", E, I, D)
    dw = _experts(rng, "q6_k", E, D, I)
    x = fp16_rows(rng, T, D)
    logits = rng.normal(0, 1, size=(T, E)).astype(np.float32)
    inds, scores = ops.moe_router_topk(_dev(logits), k, True, shared_gate=False)
    idx = inds.cpu().numpy()
    sc = scores.cpu().numpy()
    h = ops.moe_glu_gather_kq(_dev(x), _dev(gw), _dev(uw), "q4_k", inds, act=act)
    assert h.dtype == torch.float32 and tuple(h.shape) == (T, k, I)
    g_deq = okq.dequantize(gw, "q4_k").astype(np.float64)
    u_deq = okq.dequantize(uw, "q4_k").astype(np.float64)
    d_deq = okq.dequantize(dw, "q6_k").astype(np.float64)
    xf = x.astype(np.float64)

    def actf(z):
        if act == "silu":
            return z / (1 + np.exp(-z))
        return 0.5 * z * (1 + np.tanh(0.7978845608028654 * (z + 0.044715 * z ** 3)))

    href = np.stack([[actf(g_deq[idx[t, s]] @ xf[t]) * (u_deq[idx[t, s]] @ xf[t]) for s in range(k)]
                     for t in range(T)])
    assert okq.max_rel(h.cpu().numpy(), href) <= TOL
    y = ops.gather_qmv_kq(h, _dev(dw), "q6_k", inds)
    yref = np.stack([[d_deq[idx[t, s]] @ href[t, s] for s in range(k)] for t in range(T)])
    assert okq.max_rel(y.cpu().numpy(), yref) <= TOL
    mixed = ops.gather_qmv_mix_ns_kq(h, _dev(dw), "q6_k", inds, scores)
    mref = np.einsum("tk,tkn->tn", sc.astype(np.float64), yref)
    assert okq.max_rel(mixed.cpu().numpy(), mref) <= TOL
    # mix == sum over slots of the per-pair outputs (fp32, in order)
    manual = (y.cpu().numpy() * sc[..., None]).sum(1)
    assert np.allclose(mixed.cpu().numpy(), manual, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("gcodec,dcodec,D,I,E,T,k", [
    ("q4_k", "q6_k", 2048, 768, 16, 32, 8),      # C4 shapes: GLU at K = 8 super-blocks, down at K = 3
    ("q4_k", "q6_k", 1024, 256, 4, 40, 4),       # segments past 16 rows: 40 rows per expert, three chunks
    ("iq2_xxs", "iq2_xxs", 7168, 256, 6, 8, 4),  # C5 gate|up K = 28 super-blocks, down K = 256
    ("q6_k", "iq2_xxs", 3072, 512, 8, 5, 8),     # K = 12 super-blocks; every expert touched
])
def test_streaming_gather_matches_tile_gather(gcodec, dcodec, D, I, E, T, k, monkeypatch):
    """The streaming gather (every form forced, GMLX_KQ_SGATHER=2) against
    the per-tile gather kernels (=0) and the fp64 oracle: the GLU gather then
    the per-pair down gather, with one never-routed pair (zeros)."""
    from gmlx_amd import ops
    rng = np.random.default_rng(D + I + E)
    gw = _experts(rng, gcodec, E, I, D)
    uw = _experts(rng, gcodec, E, I, D)
    dw = _experts(rng, dcodec, E, D, I)
    x = fp16_rows(rng, T, D)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    idx[-1, 0] = E + 3  # never routed
    outs = {}
    for mode in ("stream", "tile"):
        monkeypatch.setenv("GMLX_KQ_SGATHER", "2" if mode == "stream" else "0")
        h = ops.moe_glu_gather_kq(_dev(x), _dev(gw), _dev(uw), gcodec, _dev(idx))
        y = ops.gather_qmv_kq(h, _dev(dw), dcodec, _dev(idx))
        outs[mode] = (h.cpu().numpy(), y.float().cpu().numpy())
    g_deq = okq.dequantize(gw, gcodec).astype(np.float64)
    u_deq = okq.dequantize(uw, gcodec).astype(np.float64)
    d_deq = okq.dequantize(dw, dcodec).astype(np.float64)
    xf = x.astype(np.float64)
    silu = lambda z: z / (1 + np.exp(-z))
    href = np.zeros((T, k, I))
    for t in range(T):
        for s_ in range(k):
            e = idx[t, s_]
            if e < E:
                href[t, s_] = silu(g_deq[e] @ xf[t]) * (u_deq[e] @ xf[t])
    for mode, (h, y) in outs.items():
        assert np.all(h[-1, 0] == 0) and np.all(y[-1, 0] == 0), mode
        assert okq.max_rel(h, href) <= TOL, (mode, okq.max_rel(h, href))
        yref = np.stack([[d_deq[idx[t, s_]] @ h[t, s_] if idx[t, s_] < E else np.zeros(D) for s_ in range(k)]
                         for t in range(T)])
        assert okq.max_rel(y, yref) <= TOL, (mode, okq.max_rel(y, yref))
    assert okq.max_rel(outs["stream"][0], outs["tile"][0]) <= TOL


def test_router_topk_matches_numpy():
    from gmlx_amd import ops
    rng = np.random.default_rng(4)
    for E, k, norm in [(128, 8, True), (256, 8, False), (60, 4, True)]:
        logits = rng.normal(0, 1, size=(17, E)).astype(np.float32)
        inds, scores = ops.moe_router_topk(_dev(logits), k, norm, shared_gate=False)
        p = np.exp(logits - logits.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        order = np.argsort(-p, axis=-1, kind="stable")[:, :k]
        assert np.array_equal(inds.cpu().numpy(), order)
        sel = np.take_along_axis(p, order, -1)
        if norm:
            sel = sel / sel.sum(-1, keepdims=True)
        assert np.allclose(scores.cpu().numpy(), sel, rtol=1e-5, atol=1e-7)


def test_out_of_range_expert_gives_zeros():
    from gmlx_amd import ops
    rng = np.random.default_rng(5)
    w = _experts(rng, "q4_k", 4, 32, 256)
    x = fp16_rows(rng, 3, 256)
    idx = np.array([[0, 9], [1, 2], [-1, 3]], np.int32)
    got = ops.gather_qmm(_dev(x), _dev(w), None, "q4_k", indices=_dev(idx)).float().cpu().numpy()
    assert np.all(got[0, 1] == 0) and np.all(got[2, 0] == 0)
    deq = okq.dequantize(w, "q4_k").astype(np.float64)
    assert okq.max_rel(got[1, 0, 0], deq[1] @ x[1].astype(np.float64)) <= TOL


def test_switch_linear_module():
    from gmlx_amd.nn import KQuantSwitchLinear
    rng = np.random.default_rng(6)
    w = _experts(rng, "q6_k", 6, 64, 512)
    mod = KQuantSwitchLinear(6, 64, 512, False, "q6_k").cuda()
    mod.weight.copy_(_dev(w))
    x = fp16_rows(rng, 4, 512)
    idx = np.array([[0, 5], [1, 1 + 1], [3, 4], [5, 0]], np.int32)
    got = mod(_dev(x).reshape(4, 1, 1, 512), _dev(idx)).float().cpu().numpy()
    deq = okq.dequantize(w, "q6_k").astype(np.float64)
    ref = np.stack([[deq[idx[t, s]] @ x[t].astype(np.float64) for s in range(2)] for t in range(4)])
    assert okq.max_rel(got[:, :, 0], ref) <= TOL


@pytest.mark.parametrize("codec,scodec,T,k,E", [("q4_k", None, 5, 4, 16), ("q4_k", "q6_k", 3, 8, 64),
                                                  ("iq2_xxs", None, 8, 8, 32), ("q6_k", "q4_k", 1, 2, 4)])
def test_shared_expert_glu_and_mix(codec, scodec, T, k, E):
    """moe_glu_gather_shexp_kq / gather_qmv_mix_kq: the shared expert in slot
    k of h and of the mix (gmlx/modules.py:571-584, 777-787), a different
    codec for the shared matrices included; routed slots equal the plain
    fused ops' results."""
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(T * 100 + k)
    D, I = 512, 256
    sc_codec = scodec or codec
    gw, uw = _experts(rng, codec, E, I, D), _experts(rng, codec, E, I, D)
    dw = _experts(rng, codec, E, D, I)
    sg, su = _experts(rng, sc_codec, 1, I, D)[0], _experts(rng, sc_codec, 1, I, D)[0]
    sd = _experts(rng, sc_codec, 1, D, I)[0]
    x = fp16_rows(rng, T, D)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    sc = rng.uniform(0.05, 1.0, size=(T, k + 1)).astype(np.float32)
    kw = {"shexp_kquant_type": scodec} if scodec else {}
    h = ops.moe_glu_gather_shexp_kq(_dev(x), _dev(gw), _dev(uw), _dev(sg), _dev(su), codec, _dev(idx), act="silu",
                                    **kw)
    assert h.dtype == torch.float32 and tuple(h.shape) == (T, k + 1, I)
    deq = lambda w, c: okq.dequantize(w, c).astype(np.float64)  # noqa: E731
    G, U, Dd = deq(gw, codec), deq(uw, codec), deq(dw, codec)
    SG, SU, SD = deq(sg, sc_codec), deq(su, sc_codec), deq(sd, sc_codec)
    xf = x.astype(np.float64)
    silu = lambda z: z / (1 + np.exp(-z))  # noqa: E731
    href = np.stack([[silu(G[idx[t, s]] @ xf[t]) * (U[idx[t, s]] @ xf[t]) for s in range(k)]
                     + [silu(SG @ xf[t]) * (SU @ xf[t])] for t in range(T)])
    assert okq.max_rel(h.cpu().numpy(), href) <= TOL
    routed = ops.moe_glu_gather_kq(_dev(x), _dev(gw), _dev(uw), codec, _dev(idx), act="silu")
    assert torch.equal(h[:, :k], routed)           # same kernel, same bits
    y = ops.gather_qmv_mix_kq(h, _dev(dw), _dev(sd), codec, _dev(idx), _dev(sc), **kw)
    assert tuple(y.shape) == (T, D) and y.dtype == torch.float32
    hh = h.cpu().numpy().astype(np.float64)
    yref = np.stack([sum(sc[t, s] * (Dd[idx[t, s]] @ hh[t, s]) for s in range(k)) + sc[t, k] * (SD @ hh[t, k])
                     for t in range(T)])
    assert okq.max_rel(y.cpu().numpy(), yref) <= TOL


@pytest.mark.parametrize("codec", ["q4_k", "iq2_xxs"])
@pytest.mark.parametrize("wave_nb", ["32", "0"])
def test_glu_gather_long_rows_both_forms(codec, wave_nb, monkeypatch):
    """GLU gather at K = 7168 (28 super-blocks per row, the C5 gate|up
    geometry) through one wave per tile (the form large decode batches take)
    and through K split over the workgroup's waves, against fp64."""
    from gmlx_amd import ops
    monkeypatch.setenv("GMLX_KQ_GATHER_WAVE_NB", wave_nb)
    rng = np.random.default_rng(29)
    E, D, I, T, k = 6, 7168, 48, 3, 2
    gw = _experts(rng, codec, E, I, D)
    uw = _experts(rng, codec, E, I, D)
    x = fp16_rows(rng, T, D)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    h = ops.moe_glu_gather_kq(_dev(x), _dev(gw), _dev(uw), codec, _dev(idx), act="silu")
    g_deq = okq.dequantize(gw, codec).astype(np.float64)
    u_deq = okq.dequantize(uw, codec).astype(np.float64)
    xf = x.astype(np.float64)
    silu = lambda z: z / (1 + np.exp(-z))  # noqa: E731
    href = np.stack([[silu(g_deq[idx[t, s]] @ xf[t]) * (u_deq[idx[t, s]] @ xf[t]) for s in range(k)]
                     for t in range(T)])
    assert okq.max_rel(h.cpu().numpy(), href) <= TOL


ROUTER_CASES = [
    # (E, k, norm, shared_gate, scoring, bias, per_expert_scale, scale, logits dtype)
    (128, 8, True, True, "softmax", False, False, 1.0, "float32"),     # gmlx/modules.py:750-752
    (64, 4, False, True, "softmax", False, False, 1.0, "bfloat16"),
    (256, 8, True, False, "sqrtsoftplus", True, False, 2.5, "float32"),  # deepseek_v4_model.py:1179-1187
    (128, 8, True, False, "softmax", False, True, 1.0, "bfloat16"),    # gemma4, modules.py:1043-1046
    (60, 6, True, False, "sigmoid", True, True, 1.5, "float16"),
    (1024, 32, False, False, "softmax", False, False, 1.0, "float32"),
]


@pytest.mark.parametrize("E,k,norm,sg,scoring,use_bias,use_pes,scale,ldt", ROUTER_CASES)
def test_router_options_match_oracle(E, k, norm, sg, scoring, use_bias, use_pes, scale, ldt):
    """moe_router_topk's keywords against the fp64 stock forms
    (oracle/moe.py): picks exactly, weights within fp32 rounding."""
    import torch
    from gmlx_amd import ops
    from oracle import moe as omoe
    rng = np.random.default_rng(E + k)
    T = 19
    tdt = getattr(torch, ldt)
    logits = torch.from_numpy(rng.normal(0, 1.5, size=(T, E + sg)).astype(np.float32)).to(tdt)
    bias = torch.from_numpy(rng.normal(0, 0.3, size=E).astype(np.float32)) if use_bias else None
    pes = torch.from_numpy(rng.uniform(0.5, 2.0, size=E).astype(np.float32)).to(torch.bfloat16) if use_pes else None
    inds, w = ops.moe_router_topk(logits.cuda(), k, norm, shared_gate=sg, scoring=scoring, scale=scale,
                                  bias=None if bias is None else bias.cuda(),
                                  per_expert_scale=None if pes is None else pes.cuda())
    assert tuple(inds.shape) == (T, k) and tuple(w.shape) == (T, k + sg)
    ri, rw = omoe.router_topk(logits.float().numpy(), k, norm, shared_gate=sg, scoring=scoring, scale=scale,
                              bias=None if bias is None else bias.numpy(),
                              per_expert_scale=None if pes is None else pes.float().numpy())
    assert np.array_equal(inds.cpu().numpy(), ri)
    assert np.allclose(w.cpu().numpy(), rw, rtol=3e-6, atol=1e-7)


@pytest.mark.parametrize("gather", ["stream", "tile"])
@pytest.mark.parametrize("seed", [11, 12, 13, 14])
@pytest.mark.parametrize("act,limit", [("silu_limit", 0.3), ("swiglu_clamp", 0.35), ("silu_limit", 1e4)])
def test_glu_limit_acts_and_biases(act, limit, seed, gather, monkeypatch):
    """silu_limit (gmlx/deepseek_v4_model.py:740-744) and the clamped,
    biased SwiGLU (gmlx/minimax_m3_model.py:134-138) epilogues, a limit small
    enough that the clamps bite, on the streaming gather and the per-tile
    gather kernels, then the down gather with its output bias
    (gather_qmv_kq(bias=), gmlx/modules.py:595-597), against fp64 by the
    reference's metric (max |err| / max |ref|, tests/test_ragged_decode.py:78-81)."""
    import torch
    from gmlx_amd import ops
    from oracle import moe as omoe
    monkeypatch.setenv("GMLX_KQ_SGATHER", "2" if gather == "stream" else "0")
    rng = np.random.default_rng(seed)
    E, D, I, T, k = 8, 512, 96, 6, 3
    gw, uw = _experts(rng, "q4_k", E, I, D), _experts(rng, "q4_k", E, I, D)
    dw = _experts(rng, "q6_k", E, D, 256)  # the down projection below runs on a 256-wide h
    x = fp16_rows(rng, T, D)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    kw = {"limit": limit}
    gb = ub = None
    if act == "swiglu_clamp":
        gb = rng.normal(0, 0.2, size=(E, I)).astype(np.float32)
        ub = rng.normal(0, 0.2, size=(E, I)).astype(np.float32)
        kw.update(alpha=1.702, gate_bias=_dev(gb), up_bias=_dev(ub))
    h = ops.moe_glu_gather_kq(_dev(x), _dev(gw), _dev(uw), "q4_k", _dev(idx), act=act, **kw)
    G = okq.dequantize(gw, "q4_k").astype(np.float64)
    U = okq.dequantize(uw, "q4_k").astype(np.float64)
    xf = x.astype(np.float64)
    href = np.stack([[omoe.glu(G[e] @ xf[t], U[e] @ xf[t], act, limit=limit, alpha=1.702,
                               gate_bias=None if gb is None else gb[e], up_bias=None if ub is None else ub[e])
                      for e in idx[t]] for t in range(T)])
    assert okq.max_rel(h.cpu().numpy(), href) <= TOL, okq.max_rel(h.cpu().numpy(), href)
    if limit < 1:  # the clamps were reached
        g_all = np.stack([[G[e] @ xf[t] for e in idx[t]] for t in range(T)])
        assert (np.abs(g_all) > limit).mean() > 0.05
    # down projection on a 256-wide h (whole Q6_K blocks) with an output bias
    h2 = torch.from_numpy(rng.normal(0, 1, size=(T, k, 256)).astype(np.float32)).cuda()
    db = rng.normal(0, 0.5, size=(E, D)).astype(np.float32)
    y = ops.gather_qmv_kq(h2, _dev(dw), "q6_k", _dev(idx), bias=_dev(db))
    Dn = okq.dequantize(dw, "q6_k").astype(np.float64)
    hh = h2.cpu().numpy().astype(np.float64)
    yref = np.stack([[Dn[e] @ hh[t, s] + db[e] for s, e in enumerate(idx[t])] for t in range(T)])
    assert okq.max_rel(y.cpu().numpy(), yref) <= TOL


def test_route_reused_once_then_recomputed():
    """A GLU gather leaves its routing for the down gather over the same idx;
    an in-place change of idx (a new version) routes afresh."""
    from gmlx_amd import ops
    rng = np.random.default_rng(12)
    E, D, I, T, k = 10, 256, 256, 4, 2
    gw, uw = _experts(rng, "q4_k", E, I, D), _experts(rng, "q4_k", E, I, D)
    dw = _experts(rng, "q4_k", E, D, I)
    x = fp16_rows(rng, T, D)
    idx_np = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    idx = _dev(idx_np)
    G, U, Dn = (okq.dequantize(w, "q4_k").astype(np.float64) for w in (gw, uw, dw))
    xf = x.astype(np.float64)
    for step in range(3):
        if step:
            idx_np = (idx_np + 3) % E
            idx.copy_(_dev(idx_np))            # in place: bumps the version counter
        h = ops.moe_glu_gather_kq(_dev(x), _dev(gw), _dev(uw), "q4_k", idx)
        y = ops.gather_qmv_kq(h, _dev(dw), "q4_k", idx)
        href = np.stack([[omoe_silu(G[e] @ xf[t]) * (U[e] @ xf[t]) for e in idx_np[t]] for t in range(T)])
        yref = np.stack([[Dn[e] @ href[t, s] for s, e in enumerate(idx_np[t])] for t in range(T)])
        assert okq.max_rel(h.cpu().numpy(), href) <= TOL
        assert okq.max_rel(y.cpu().numpy(), yref) <= TOL


def omoe_silu(z):
    return z / (1 + np.exp(-z))


def test_wide_range_activations_through_the_moe_layer():
    """bf16 activations with entries of 1e5 into the fused GLU gather, and its
    fp32 outputs (above fp16's 65504, and rows near 1e-12) into the down
    gather: both prepare their rows as fp16 with a power of two per row and
    scale the fp32 results back before the GLU / the store, so every pair
    row matches the fp64 reference on its own scale."""
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(12)
    E, D, I, T, k = 8, 512, 256, 4, 2
    gw = _experts(rng, "q4_k", E, I, D)
    uw = _experts(rng, "q4_k", E, I, D)
    dw = _experts(rng, "q6_k", E, D, I)
    x = rng.normal(0, 1, size=(T, D)).astype(np.float32)
    x[0] *= 1e5
    x[1] *= 1e-6
    xb = torch.from_numpy(x).to(torch.bfloat16)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    inds = _dev(idx)
    h = ops.moe_glu_gather_kq(xb.cuda(), _dev(gw), _dev(uw), "q4_k", inds, act="silu")
    g_deq = okq.dequantize(gw, "q4_k").astype(np.float64)
    u_deq = okq.dequantize(uw, "q4_k").astype(np.float64)
    d_deq = okq.dequantize(dw, "q6_k").astype(np.float64)
    xf = xb.float().numpy().astype(np.float64)

    def silu(z):
        return z / (1 + np.exp(-np.clip(z, -700, 700)))

    href = np.stack([[silu(g_deq[idx[t, s]] @ xf[t]) * (u_deq[idx[t, s]] @ xf[t]) for s in range(k)]
                     for t in range(T)])
    hg = h.cpu().numpy()
    assert np.abs(hg[0]).max() > 65504.0        # the GLU output row leaves fp16's range
    for t in range(T):
        for s in range(k):
            assert okq.max_rel(hg[t, s], href[t, s]) <= TOL, (t, s)
    # fp32 rows far outside fp16's range into the per-pair down gather
    hin = href.astype(np.float32)
    hin[2, 0] *= 1e-10
    y = ops.gather_qmv_kq(_dev(hin), _dev(dw), "q6_k", inds)
    yg = y.cpu().numpy()
    hf = hin.astype(np.float64)
    for t in range(T):
        for s in range(k):
            want = d_deq[idx[t, s]] @ hf[t, s]
            assert okq.max_rel(yg[t, s], want) <= TOL, (t, s)


def test_biased_switch_linear_module():
    """KQuantSwitchLinear with a bias: each pair adds its expert's fp32 bias
    row in the kernel's epilogue."""
    import torch
    from gmlx_amd.nn import KQuantSwitchLinear
    rng = np.random.default_rng(16)
    w = _experts(rng, "q4_k", 5, 48, 512)
    mod = KQuantSwitchLinear(5, 48, 512, True, "q4_k").cuda()
    mod.weight.copy_(_dev(w))
    b = rng.normal(0, 1, size=(5, 48)).astype(np.float32)
    mod.bias.copy_(torch.from_numpy(b))
    x = fp16_rows(rng, 3, 512)
    idx = np.array([[0, 4], [2, 2 + 1], [4, 1]], np.int32)
    got = mod(_dev(x).reshape(3, 1, 1, 512), _dev(idx)).float().cpu().numpy()
    deq = okq.dequantize(w, "q4_k").astype(np.float64)
    ref = np.stack([[deq[idx[t, s]] @ x[t].astype(np.float64) + b[idx[t, s]] for s in range(2)] for t in range(3)])
    assert okq.max_rel(got[:, :, 0], ref) <= TOL


@pytest.mark.parametrize("codec,dtype_name", [("q4_k", "bfloat16"), ("q6_k", "float16"), ("iq2_xxs", "float32")])
def test_kquant_embedding(codec, dtype_name):
    """KQuantEmbedding: forward(ids) gives the GGML dequantization of the ids'
    rows (bit-exact in fp32, one rounding otherwise); as_linear(x) is the
    tied head x . dequant(W)^T."""
    import torch
    from gmlx_amd.nn import KQuantEmbedding
    rng = np.random.default_rng(21)
    V, D = 300, 512
    if codec == "iq2_xxs":
        wire = okq.random_valid_blocks(rng, codec, V * D // 256).reshape(V, -1)
    else:
        wire = quantized_weights(rng, codec, V, D)
    tdt = getattr(torch, dtype_name)
    emb = KQuantEmbedding(V, D, codec, out_dtype=tdt).cuda()
    emb.weight.copy_(_dev(wire))
    ids = rng.integers(0, V, size=(2, 7))
    got = emb(torch.from_numpy(ids).cuda())
    assert got.dtype == tdt and tuple(got.shape) == (2, 7, D)
    deq = okq.dequantize(wire, codec)                                  # fp32, the GGML definition
    want = torch.from_numpy(deq[ids.reshape(-1)].reshape(2, 7, D)).to(tdt)
    assert torch.equal(got.cpu(), want)
    x = fp16_rows(rng, 3, D)
    logits = emb.as_linear(_dev(x)).float().cpu().numpy()
    ref = x.astype(np.float64) @ deq.astype(np.float64).T
    assert okq.max_rel(logits, ref) <= TOL



@pytest.mark.parametrize("dcodec,T,k,E,I,N,bad", [
    ("q6_k", 32, 8, 128, 768, 2048, False),   # C4's down
    ("iq2_xxs", 8, 8, 64, 2048, 1024, False),
    ("q4_k", 5, 4, 6, 256, 200, True),        # a partial last tile; out-of-range experts give zero rows
    ("q6_k", 40, 8, 16, 512, 2048, False),
    ("q4_k", 3, 2, 4, 4096, 64, True),        # 16 super-blocks per row: the split-K gather
])
@pytest.mark.parametrize("hdt", ["float32", "float16"])
def test_down_gather_with_mix_equals_two_steps(dcodec, T, k, E, I, N, bad, hdt):
    """gather_qmv_mix_ns_kq bitwise equal to the per-pair gather followed by
    the slot-ordered fp32 mix written out in torch; repeated calls and graph
    replays bitwise equal; and within tolerance of fp64
    (gmlx/modules.py:591-593)."""
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(T * 31 + k + E + I)
    dw = _dev(_experts(rng, dcodec, E, N, I))
    idx_np = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    if bad:
        idx_np[0, 1], idx_np[-1, 0] = -1, E + 3
    idx = _dev(idx_np)
    sc = torch.from_numpy(rng.uniform(0.1, 1.0, size=(T, k)).astype(np.float32)).cuda()
    h = torch.from_numpy(rng.normal(0, 1, size=(T, k, I)).astype(np.float32)).to(getattr(torch, hdt)).cuda()
    print(f"mix {dcodec} T={T} k={k} E={E} I={I} N={N} {hdt}", flush=True)
    yp = ops.gather_qmv_kq(h, dw, dcodec, idx)                       # (T, k, N) fp32
    want = torch.zeros((T, N), dtype=torch.float32, device="cuda")
    for s in range(k):
        want = want + sc[:, s:s + 1] * yp[:, s]
    outs = [ops.gather_qmv_mix_ns_kq(h, dw, dcodec, idx, sc) for _ in range(3)]
    for o in outs:
        assert torch.equal(o, want)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        og = ops.gather_qmv_mix_ns_kq(h, dw, dcodec, idx, sc)
    for _ in range(3):
        ops.gather_qmv_mix_ns_kq(h, dw, dcodec, idx, sc)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(og, want)
    D = okq.dequantize(dw.cpu().numpy(), dcodec).reshape(E, N, I).astype(np.float64)
    hf = h.double().cpu().numpy()
    ref = np.zeros((T, N))
    for t in range(T):
        for s, e in enumerate(idx_np[t]):
            if 0 <= e < E:
                ref[t] += float(sc[t, s]) * (D[e] @ hf[t, s])
    assert okq.max_rel(want.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("gcodec,dcodec", [("q4_k", "q6_k"), ("iq2_xxs", "iq2_xxs")])
def test_glu_gather_fp16_h_skips_the_prepare_pass(gcodec, dcodec):
    """moe_glu_gather_kq(out_dtype=float16): h is the fp32 h rounded to fp16,
    bitwise, on both gather forms' codecs; the layer through the down gather
    and mix matches the fp32-h layer (whose down gather prepares its rows)
    and the fp64 reference within tolerance."""
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(31)
    E, D, I, T, k = 32, 2048, 768, 16, 8
    if gcodec == "iq2_xxs":
        gw, uw, dw = (okq.random_valid_blocks(rng, "iq2_xxs", E * n * kk // 256).reshape(E, n, -1)
                      for n, kk in ((I, D), (I, D), (D, I)))
    else:
        gw, uw, dw = _experts(rng, gcodec, E, I, D), _experts(rng, gcodec, E, I, D), _experts(rng, dcodec, E, D, I)
    x = fp16_rows(rng, T, D)
    logits = rng.normal(0, 1, size=(T, E)).astype(np.float32)
    inds, scores = ops.moe_router_topk(_dev(logits), k, True, shared_gate=False)
    args = (_dev(x), _dev(gw), _dev(uw), gcodec, inds)
    h32 = ops.moe_glu_gather_kq(*args)
    h16 = ops.moe_glu_gather_kq(*args, out_dtype=torch.float16)
    assert h16.dtype == torch.float16 and h16.shape == h32.shape
    assert torch.equal(h16, h32.to(torch.float16))
    dd = _dev(dw)
    y32 = ops.gather_qmv_mix_ns_kq(h32, dd, dcodec, inds, scores).cpu().numpy()
    y16 = ops.gather_qmv_mix_ns_kq(h16, dd, dcodec, inds, scores).cpu().numpy()
    assert okq.max_rel(y16, y32) <= TOL
    idx, sc = inds.cpu().numpy(), scores.cpu().numpy().astype(np.float64)
    d_deq = okq.dequantize(dw.reshape(-1, dw.shape[-1]), dcodec).reshape(E, D, I).astype(np.float64)
    hf = h16.float().cpu().numpy().astype(np.float64)
    yref = np.stack([sum(sc[t, s] * (d_deq[idx[t, s]] @ hf[t, s]) for s in range(k)) for t in range(T)])
    assert okq.max_rel(y16, yref) <= TOL
    with pytest.raises(ValueError):
        ops.moe_glu_gather_kq(*args, out_dtype=torch.int32)
