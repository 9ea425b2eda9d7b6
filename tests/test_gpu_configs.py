"""Parity at the full C3 / C4 / C5 workloads, through the default launch plans (no
environment overrides), against the fp64 oracle:

  C3  ragged GQA decode attention: 32 q heads / 8 kv heads / D 128, B = 16
      rows with the seed-0 log-uniform lengths (1037 .. 95651 tokens), per-row
      KV slabs, scale 1/sqrt(128): every row and head (the reference's
      construction, tests/test_ragged_decode.py:48-81);
  C4  MoE layer, 128 experts top-8, D 2048, I 768, 32 tokens, gate/up Q4_K
      and down Q6_K quantised from N(0, 0.02): router, fused GLU gather and
      the down gather with the routing mix;
  C5  MoE layer, 256 experts top-8, D 7168, I 2048, 8 tokens, IQ2_XXS:
      the touched experts quantised by kq_quantize from N(0, 0.02).
"""
import math

import numpy as np
import pytest

from helpers import TOL
from oracle import attention as oat
from oracle import kquant as okq
from oracle import moe as omoe

pytestmark = pytest.mark.gpu

C3_LENS = [22517, 3791, 1249, 1109, 52970, 85835, 19436, 35277, 14316, 95651, 53638, 1037, 65619, 1205, 35305,
           2401]


def test_c3_lengths_are_the_seed0_draw():
    rng = np.random.default_rng(0)
    lens = np.exp(rng.uniform(math.log(1024), math.log(131072), 16)).astype(np.int64)
    assert lens.tolist() == C3_LENS


def test_c3_ragged_attention_full():
    import torch
    from gmlx_amd import ops
    Hq, Hkv, D, B = 32, 8, 128, 16
    lens = C3_LENS
    offs = np.concatenate([[0], np.cumsum([Hkv * L * D for L in lens])[:-1]]).astype(np.int64)
    total = int(sum(Hkv * L * D for L in lens))
    gen = torch.Generator(device="cuda").manual_seed(0)
    k = torch.randn(total, generator=gen, device="cuda", dtype=torch.float32).half()
    v = torch.randn(total, generator=gen, device="cuda", dtype=torch.float32).half()
    q = torch.randn((B, Hq, D), generator=gen, device="cuda", dtype=torch.float32).half()
    out = ops.sdpa_decode_slabs(q, k, v, offs.tolist(), lens, Hkv, D ** -0.5)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    qn = q.float().cpu().numpy()
    worst = 0.0
    for b in range(B):
        o, L = int(offs[b]), lens[b]
        kb = k[o:o + Hkv * L * D].float().cpu().numpy().reshape(Hkv, L, D)
        vb = v[o:o + Hkv * L * D].float().cpu().numpy().reshape(Hkv, L, D)
        ref = oat.row_attention(qn[b], kb, vb, D ** -0.5)
        err = okq.max_rel(got[b], ref)
        worst = max(worst, err)
        assert err <= TOL, f"row {b} (len {L}): max-rel {err:.3e}"
    print(f"C3 worst row max-rel {worst:.3e}")


def _quantized_stack(torch, ops, gen, E, N, K, codec, only=None):
    """[E, N, K] wire stack from N(0, 0.02) weights quantised on the GPU by
    kq_quantize (byte-identical to the oracle's quantizer, checked in
    test_gpu_dequant_quantize).  With `only`, the other experts' bytes are
    zeros (they are never read)."""
    from oracle.kquant import BLOCK_BYTES
    rb = K // 256 * BLOCK_BYTES[codec]
    out = torch.zeros((E, N, rb), dtype=torch.uint8, device="cuda")
    for e in (range(E) if only is None else sorted(only)):
        w = torch.randn((N, K), generator=gen, device="cuda") * 0.02
        out[e].copy_(ops.quantize(w, codec)[0])
    return out


def _moe_layer_check(E, D, I, topk, T, cgu, cd, only_touched):
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(0)
    logits = rng.normal(0.0, 1.0, size=(T, E)).astype(np.float32)
    x = rng.normal(0.0, 1.0, size=(T, D)).astype(np.float16)
    inds, w = ops.moe_router_topk(torch.from_numpy(logits).cuda(), topk, True, shared_gate=False)
    ri, rw = omoe.router_topk(logits, topk, True, shared_gate=False)
    idx = inds.cpu().numpy()
    assert np.array_equal(idx, ri)
    assert np.allclose(w.cpu().numpy(), rw, rtol=2e-6, atol=1e-7)
    touched = set(np.unique(idx).tolist()) if only_touched else None
    gen = torch.Generator(device="cuda").manual_seed(0)
    g = _quantized_stack(torch, ops, gen, E, I, D, cgu, touched)
    u = _quantized_stack(torch, ops, gen, E, I, D, cgu, touched)
    d = _quantized_stack(torch, ops, gen, E, D, I, cd, touched)
    xd = torch.from_numpy(x).cuda()
    h = ops.moe_glu_gather_kq(xd, g, u, cgu, inds)
    y = ops.gather_qmv_mix_ns_kq(h, d, cd, inds, w)
    torch.cuda.synchronize()
    h_got, y_got = h.cpu().numpy(), y.cpu().numpy()
    # fp64 over the touched experts, one expert at a time
    xf = x.astype(np.float64)
    wts = w.cpu().numpy().astype(np.float64)
    h_ref = np.zeros((T, topk, I))
    y_ref = np.zeros((T, D))
    for e in np.unique(idx):
        G = okq.dequantize(g[e].cpu().numpy(), cgu).astype(np.float64)
        U = okq.dequantize(u[e].cpu().numpy(), cgu).astype(np.float64)
        Dn = okq.dequantize(d[e].cpu().numpy(), cd).astype(np.float64)
        for t, s in zip(*np.nonzero(idx == e)):
            h_ref[t, s] = omoe.glu(G @ xf[t], U @ xf[t], "silu")
            y_ref[t] += wts[t, s] * (Dn @ h_ref[t, s])
    eh, ey = okq.max_rel(h_got, h_ref), okq.max_rel(y_got, y_ref)
    print(f"{len(np.unique(idx))} touched experts: h max-rel {eh:.3e}, y max-rel {ey:.3e}")
    assert eh <= TOL and ey <= TOL


def test_c4_moe_layer_full():
    _moe_layer_check(128, 2048, 768, 8, 32, "q4_k", "q6_k", only_touched=False)


def test_c5_moe_layer_full():
    _moe_layer_check(256, 7168, 2048, 8, 8, "iq2_xxs", "iq2_xxs", only_touched=True)
