#!/usr/bin/env python3
"""Benchmark of the K-quant batched-decode hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch B]

Headline (workload C2): one decode step through the linear layers of a
Qwen3-8B Q4_K_M stack -- 36 layers, each q 4096x4096, k 1024x4096,
o 4096x4096, gate/up 12288x4096 in Q4_K and v 1024x4096, down 4096x12288 in
Q6_K -- at B rows of fp16 activations.  Per layer the launches follow the
decode data flow: q|k|v grouped (one launch), o, gate|up grouped, down.
Every layer has its own weight bytes (4.41 GB per step), so nothing is served
from the 256 MB MALL.  A step is replayed from a HIP graph (the launches are
5-10 us each; eager Python launching would measure the host).

`value` = algorithmic weight + activation bytes per step / step time (GB/s).
The `roofline` object is for the kernel family with the largest share of the
step (its launches of the step alone, replayed from a graph): achieved =
algorithmic bytes per launch / average launch duration, both over the timed
region; `traffic` = HBM bytes per launch of the same family from the
FETCH_SIZE / WRITE_SIZE counters.  Extra fields: the per-B sweep (B = 1..64, same
stack), ragged GQA decode attention on workload C3 (KV GB/s, KV tokens/s),
cascade shared-prefix decode attention beside the ragged kernel on the same
buffer, one MoE decode layer on workloads C4 and C5 (GB/s over the touched
experts' bytes) and the CPU baseline (the repository's OpenMP C restatement of the same
dequant-fused matmul, timed on a bounded sample of the same workload).

Inputs: numpy default_rng(seed) draws, N(0, 0.02) weights quantised on the GPU
by kq_quantize (byte-identical to the llama.cpp-style reference quantiser in
oracle/), fp16 N(0, 1) activations.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "Q4_K_M decode matmul GB/s (% HBM peak) at B=1..64; ragged SDPA tokens/s"

HIDDEN, INTER, LAYERS = 4096, 12288, 36
# (name, N, K, codec) of one Qwen3-8B layer under the Q4_K_M mix
LAYER = [("q", 4096, 4096, "q4_k"), ("k", 1024, 4096, "q4_k"), ("v", 1024, 4096, "q6_k"),
         ("o", 4096, 4096, "q4_k"), ("gate", INTER, 4096, "q4_k"), ("up", INTER, 4096, "q4_k"),
         ("down", 4096, INTER, "q6_k")]
BPB = {"q4_k": 144, "q6_k": 210}
C3_LENS_SEED = 0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def wire_bytes(N, K, codec):
    return N * (K // 256) * BPB[codec]


def layer_bytes(B):
    """Algorithmic bytes of one layer at B rows: weights + fp16 x in (once per
    launch) + fp16 y out."""
    return sum(launch_bytes(launch, B) for launch, _ in LAUNCHES)


# ------------------------------------------------------------------ weights

def make_stack(torch, ops, layers, seed=0):
    """`layers` distinct layers of wire bytes on the GPU.  The first layer is
    quantised from numpy draws (seed, draw order q, k, v, o, gate, up, down);
    the others are byte copies at their own addresses."""
    import numpy as np
    rng = np.random.default_rng(seed)
    base = {}
    for name, N, K, codec in LAYER:
        w = torch.from_numpy(rng.normal(0.0, 0.02, size=(N, K)).astype(np.float32)).cuda()
        base[name] = ops.quantize(w, codec)[0]
        del w
    stack = [base]
    for _ in range(layers - 1):
        stack.append({k: v.clone() for k, v in base.items()})
    torch.cuda.synchronize()
    return stack, rng


def make_inputs(torch, rng, B):
    import numpy as np
    x = torch.from_numpy(rng.normal(0.0, 1.0, size=(B, HIDDEN)).astype(np.float16)).cuda()
    xd = torch.from_numpy(rng.normal(0.0, 1.0, size=(B, INTER)).astype(np.float16)).cuda()
    return x, xd


# The launches of one layer: (name, matrices), and the kernel that serves
# each (kq_quantized_matmul_grouped's routing): at B <= 8 gate|up (six tiles
# per CU) takes the producer / consumer weight-streaming kernel (two waves copy
# whole 16-row tiles into an LDS ring with direct-to-LDS loads, eight waves
# dequantize and run the MFMA on one K-slab each), and so does down (K = 12288
# Q6_K) in six K slices of 8 super-blocks, the last slice of each tile to
# finish summing the six partial tiles; q|k|v and o (one or two tiles per CU)
# take the one-shot kernel (every wave copies one super-block column of its
# workgroup's tiles and its activation slab into LDS at entry and multiplies
# as soon as its own loads land; one barrier before the partial-tile sum; at
# 9..16 rows the activation slab is copied in two passes of 8 rows; at
# 17..32 rows two 16-row blocks run one after the other through the same
# slab, the columns staying in LDS).
# At B = 9..16 gate|up and down take the streaming kernel's 16-row forms
# (down in four K slices of 12 super-blocks).
# At B = 17..64 gate|up and down (and q|k|v past 32 rows) take the mid-batch streaming kernel
# (four waves copy each super-block of the activation rows and of a group of
# six weight tiles into an LDS ring, six waves each accumulate one tile over
# the group's K slice): gate|up unsplit (256 groups), down in five K slices,
# q|k|v in three, the last slice of each tile summing the partial tiles; o
# past 32 rows takes the 17..64-row tile kernel (one 4-wave workgroup per CU
# per weight tile); past 64 rows the general kernel.
LAUNCHES = [("qkv", ("q", "k", "v")), ("o", ("o",)), ("gate_up", ("gate", "up")), ("down", ("down",))]
CODEC = {name: codec for name, _, _, codec in LAYER}
DIMS = {name: (N, K) for name, N, K, _ in LAYER}
# kernel families, as rocprofv3 names them
KERNEL_FAMILIES = ("kq_stream_kernel", "kq_shot_kernel", "kq_mms_kernel", "kq_mv_kernel", "kq_mm_kernel",
                   "kq_dense_grouped_kernel")


def kernel_of(launch, B):
    """Kernel (with template arguments) that serves `launch` at B rows."""
    mt = 1 if B <= 16 else 2 if B <= 32 else 4
    dense = f"kq_dense_grouped_kernel<{mt}, 0, {16 if B <= 16 else 4}, {1 if B <= 16 else 2}>"
    if B > 64:
        return dense
    if B > 16:
        # up to 32 rows q|k|v and o take the one-shot kernel's 32-row form (two 16-row blocks);
        # kq_mms_kernel<codec (12 Q4_K, 14 Q6_K, 127 both), 16-row blocks, tiles per group, ring slots>
        # (q|k|v in 3 K slices, down in 5, gate|up unsplit); o: kq_mm_kernel<codec set (0 Q4_K),
        # 16-row blocks, fp16, tiles per group>
        if B <= 32 and launch in ("qkv", "o"):
            return "kq_shot_kernel<16, 32>"
        return {"qkv": f"kq_mms_kernel<127, {mt}, 6, {4 if mt == 2 else 2}>", "o": f"kq_mm_kernel<0, {mt}, 0, 1>",
                "gate_up": f"kq_mms_kernel<12, {mt}, 6, {4 if mt == 2 else 3}>",
                "down": f"kq_mms_kernel<14, {mt}, 6, {4 if mt == 2 else 2}>"}[launch]
    if launch == "gate_up":  # kq_stream_kernel<codec, blocks per consumer, consumers, slots, rows>
        return f"kq_stream_kernel<12, 2, 8, 3, {8 if B <= 8 else 16}>"
    if B <= 16 and launch == "down":  # K = 12288 in slices, one super-block per consumer
        # up to 8 rows: six slices of 8; 9..16 rows: four slices of 12 (two ring slots)
        return "kq_stream_kernel<14, 1, 8, 3, 8>" if B <= 8 else "kq_stream_kernel<14, 1, 12, 2, 16>"
    if launch in ("qkv", "o"):  # kq_shot_kernel<super-blocks per row, activation rows>
        return f"kq_shot_kernel<16, {8 if B <= 8 else 16}>"
    raise ValueError(launch)


def family(kernel):
    return kernel.split("<")[0]


def launch_bytes(launch, B):
    """Algorithmic bytes of one launch: wire bytes + fp16 x in + fp16 y out."""
    tot = 0
    for m in dict(LAUNCHES)[launch]:
        N, K = DIMS[m]
        tot += wire_bytes(N, K, CODEC[m]) + B * N * 2
    N, K = DIMS[dict(LAUNCHES)[launch][0]]
    return tot + B * K * 2  # x read once per launch (shared by grouped problems)


def run_launch(ops, L, launch, x, xd):
    if launch == "qkv":
        return ops.quantized_matmul_grouped([(x, L["q"], "q4_k"), (x, L["k"], "q4_k"), (x, L["v"], "q6_k")])
    if launch == "o":
        return [ops.quantized_matmul(x, L["o"], None, "q4_k")]
    if launch == "gate_up":
        return ops.quantized_matmul_grouped([(x, L["gate"], "q4_k"), (x, L["up"], "q4_k")])
    return [ops.quantized_matmul(xd, L["down"], None, "q6_k")]


def spot_check_layer(torch, ops, L, x, xd, rows_per_matrix=64, seed=5):
    """max_rel of one layer's four launches at rows_per_matrix seeded weight
    rows of each matrix, against fp64 over the library's bit-exact
    dequantization of the same wire rows (kq_dequantize, pinned to the GGML
    definitions by the GPU tests)."""
    import numpy as np
    outs = {}
    for launch, mats in LAUNCHES:
        for m, y in zip(mats, run_launch(ops, L, launch, x, xd)):
            outs[m] = y.float().cpu().numpy()
    rng = np.random.default_rng(seed)
    res = {}
    for launch, mats in LAUNCHES:
        worst = 0.0
        for m in mats:
            N, K = DIMS[m]
            rows = np.sort(rng.choice(N, size=min(rows_per_matrix, N), replace=False))
            wr = ops.dequantize(L[m][torch.from_numpy(rows).cuda()], None, CODEC[m]).double().cpu().numpy()
            xin = (xd if K == INTER else x).double().cpu().numpy()
            ref = xin @ wr.T
            got = outs[m][:, rows]
            worst = max(worst, float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30)))
        res[launch] = worst
    return res


def step_fn(ops, stack, x, xd, only=None):
    """One decode step of the linear stack: 4 launches per layer (or only the
    launches named in `only`)."""
    outs = []
    for L in stack:
        outs = []
        for launch, _ in LAUNCHES:
            if only is None or launch in only:
                outs += run_launch(ops, L, launch, x, xd)
    return outs


def capture(torch, fn):
    fn()  # eager warm-up: grows the workspace outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = fn()
    torch.cuda.synchronize()
    return g, outs


def time_graph(torch, g, steps, warmup):
    """Mean ms per replay over `steps` back-to-back replays (one event pair
    around the whole timed region)."""
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps  # ms per replay


def quantiles(samples_ms):
    """Median and p10 / p90 (ms) of per-iteration timings."""
    import numpy as np
    a = np.asarray(samples_ms, np.float64)
    return {"median_ms": round(float(np.median(a)), 5), "p10_ms": round(float(np.percentile(a, 10)), 5),
            "p90_ms": round(float(np.percentile(a, 90)), 5), "n": int(a.size)}


def replay_samples(torch, g, n, flush=None):
    """Per-replay timings (ms) of n replays, each bracketed by its own event
    pair; with `flush`, a callable run before each replay outside the events
    (a write of more than twice the 256 MB MALL, so every timed replay reads
    its bytes from HBM)."""
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for a, b in ev:
        if flush is not None:
            flush()
        a.record()
        g.replay()
        b.record()
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in ev]


def mall_flush(torch):
    """A callable that overwrites 1 GiB of device memory (4x the MALL)."""
    buf = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    return lambda: buf.fill_(1)


def copy_peak(torch, nbytes=1 << 30, iters=20):
    """On-box HBM references, medians over iters with the MALL cold (each
    buffer is 4x the MALL): a device-to-device copy of nbytes (read + write
    2 nbytes), the same copy as a float32 elementwise kernel, and a read-only
    pass (sum of nbytes).  `gbs_median` is the best of them."""
    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    src.fill_(1.0)
    variants = {
        "memcpy_d2d": (lambda: dst.copy_(src), 2 * nbytes),
        "elementwise_copy": (lambda: torch.mul(src, 1.0, out=dst), 2 * nbytes),
        "read_sum": (lambda: src.sum(), nbytes),
    }
    out = {}
    for name, (fn, moved) in variants.items():
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(iters):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            e1.synchronize()
            ts.append(e0.elapsed_time(e1))
        q = quantiles(ts)
        out[name] = {"bytes_moved": moved, "gbs_median": round(moved / q["median_ms"] / 1e6, 1), **q}
    del src, dst
    torch.cuda.empty_cache()
    best = max(v["gbs_median"] for v in out.values())
    return {"gbs_median": best, "frac_of_8tbs": round(best / HBM_PEAK_GBS, 4), "variants": out,
            "what": "best of a 1 GiB device copy (memcpy, elementwise) and a 1 GiB read-only sum"}


# ---------------------------------------------------------------- attention

def c3_lengths(seed=C3_LENS_SEED, B=16):
    import numpy as np
    rng = np.random.default_rng(seed)
    return np.exp(rng.uniform(math.log(1024), math.log(131072), B)).astype(np.int64), rng


def timed_calls(torch, fn, n, flush=None):
    """Per-call timings (ms) of n eager calls, each between its own events;
    with `flush`, a MALL-overwriting write before each call, outside them."""
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for a, b in ev:
        if flush is not None:
            flush()
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in ev]


def cpu_sdpa_baseline(q, k, v, offs, lens, Hkv, scale, budget_s=6.0):
    """CPU figure beside C3: the oracle's OpenMP fp32 online-softmax ragged
    attention (oracle/kq_oracle.c kqo_ragged_attn_f32) over the whole C3
    batch (host copies of the same fp16 q, K, V), repeated until ~budget_s on
    the host threads this process may use (as cpu_baseline)."""
    import numpy as np
    from oracle import kquant as okq
    L = okq.lib()
    B, Hq, D = q.shape
    lens32 = np.ascontiguousarray(lens, dtype=np.int32)
    offs64 = np.ascontiguousarray(offs, dtype=np.int64)
    hs = lens32.astype(np.int64) * D  # one kv head's slab: len x D elements
    out = np.empty((B, Hq, D), np.float32)
    affinity = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "").strip()
    nthreads = min(affinity, int(omp)) if omp.isdigit() and int(omp) > 0 else affinity
    done, t0 = 0, time.perf_counter()
    while True:
        L.kqo_ragged_attn_f32(q.ctypes.data, k.ctypes.data, v.ctypes.data, offs64.ctypes.data, hs.ctypes.data,
                              lens32.ctypes.data, B, Hq, Hkv, D, scale, out.ctypes.data, nthreads)
        done += 1
        el = time.perf_counter() - t0
        if el >= budget_s or done >= 20:
            break
    kv_bytes = 2 * k.size * 2
    return {"kv_gbs": round(done * kv_bytes / el / 1e9, 3), "unit": "GB/s",
            "kv_tokens_per_s": round(done * int(lens.sum()) / el, 1), "cores": nthreads, "kind": "port",
            "sample": f"{done} pass(es) of the whole C3 batch ({kv_bytes / 1e9:.2f} GB of fp16 K/V), {el:.1f} s, "
                      f"oracle/kq_oracle.c kqo_ragged_attn_f32 (OpenMP, fp32 online softmax)"}


def bench_sdpa(torch, ops, iters=50, cpu=False):
    """Workload C3: 32 q heads / 8 kv heads, D 128, B 16 ragged rows in
    per-row [Hkv, len, D] slabs (offset table), fp16, scale 1/sqrt(128).
    cpu: also time the CPU restatement on the same batch (cpu_sdpa_baseline)."""
    import numpy as np
    lens, rng = c3_lengths()
    B, Hq, Hkv, D = 16, 32, 8, 128
    offs = np.concatenate([[0], np.cumsum(lens * Hkv * D)[:-1]]).astype(np.int64)
    total = int(lens.sum()) * Hkv * D
    gen = torch.Generator(device="cuda").manual_seed(0)
    k = torch.randn(total, generator=gen, device="cuda", dtype=torch.float32).half()
    v = torch.randn(total, generator=gen, device="cuda", dtype=torch.float32).half()
    q = torch.from_numpy(rng.normal(0, 1, size=(B, Hq, D)).astype(np.float16)).cuda()
    scale = 1.0 / math.sqrt(D)
    offl, lenl = offs.tolist(), lens.tolist()
    run = lambda: ops.sdpa_decode_slabs(q, k, v, offl, lenl, Hkv, scale)  # noqa: E731
    out = run()
    torch.cuda.synchronize()
    # 2.0 GB of KV per call: every call streams from HBM (8x the MALL)
    qs16 = quantiles(timed_calls(torch, run, iters))
    ms = qs16["median_ms"]
    kv_bytes = 2 * total * 2
    qo_bytes = 2 * B * Hq * D * 2
    # spot-check two heads of the shortest and longest rows against fp64
    chk = 0.0
    for b in (int(np.argmin(lens)), int(np.argmax(lens))):
        L = int(lens[b])
        for hq in (0, Hq - 1):
            h = hq // (Hq // Hkv)
            base = int(offs[b]) + h * L * D
            kb = k[base:base + L * D].view(L, D).double().cpu().numpy()
            vb = v[base:base + L * D].view(L, D).double().cpu().numpy()
            s = kb @ q[b, hq].double().cpu().numpy() * scale
            p = np.exp(s - s.max())
            ref = p @ vb / p.sum()
            got = out[b, hq].double().cpu().numpy()
            chk = max(chk, float(np.abs(got - ref).max() / np.abs(ref).max()))
    cpu_line = None
    if cpu:
        cpu_line = cpu_sdpa_baseline(q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(), offs, lens, Hkv, scale)
    # the same batch over an 8-bit affine KV cache (group 64): half the KV bytes
    q8 = {}
    kq8, vq8, scs = [], [], []
    for t in (k, v):
        g = t.view(-1, 64).float()
        lo, hi = g.min(1, keepdim=True).values, g.max(1, keepdim=True).values
        sc_ = ((hi - lo).clamp_min(1e-6) / 255.0).half()
        bi_ = lo.half()
        qv = ((g - bi_.float()) / sc_.float()).round_().clamp_(0, 255).to(torch.uint8).view(-1)
        (kq8 if t is k else vq8).append(qv)
        scs += [sc_.view(-1), bi_.view(-1)]
        del g
    del k, v
    run8 = lambda: ops.sdpa_decode_slabs(q, kq8[0], vq8[0], offl, lenl, Hkv, scale,  # noqa: E731
                                         k_scales=scs[0], k_biases=scs[1], v_scales=scs[2], v_biases=scs[3])
    qs8 = quantiles(timed_calls(torch, run8, iters))
    ms8 = qs8["median_ms"]
    q8_bytes = 2 * total + 2 * (total // 64) * 4  # values + fp16 scale and bias per 64
    q8 = {"ms": round(ms8, 4), "timing": qs8, "kv_gbs": round(q8_bytes / ms8 / 1e6, 1),
          "frac_hbm": round(q8_bytes / ms8 / 1e6 / HBM_PEAK_GBS, 4),
          "kv_tokens_per_s": round(int(lens.sum()) / ms8 * 1e3, 1), "kv_bytes": q8_bytes}
    del kq8, vq8, scs
    return {
        "q8_kv": q8,
        "workload": "C3 ragged GQA decode, 32q/8kv heads, D=128, B=16, lens log-uniform 1k..128k (seed 0), fp16",
        "kv_tokens": int(lens.sum()),
        "ms": round(ms, 4),
        "timing": qs16,
        "kv_gbs": round(kv_bytes / ms / 1e6, 1),
        "frac_hbm": round(kv_bytes / ms / 1e6 / HBM_PEAK_GBS, 4),
        "kv_tokens_per_s": round(int(lens.sum()) / ms * 1e3, 1),
        "rows_per_s": round(B / ms * 1e3, 1),
        "algorithmic_bytes": kv_bytes + qo_bytes,
        "max_rel_spot": chk,
        "cpu_baseline": cpu_line,
    }


def bench_cascade(torch, ops, iters=50):
    """Cascade shared-prefix decode (kq.sdpa_decode_gqa_cascade, the claim of
    gmlx/cascade_sdpa.py:136-260): B = 8 sequences share a P = 16384-token
    prefix, then 512 private tokens each after ragged left pads; qL 1,
    32 q / 8 kv heads, D 128, fp16.  Timed beside the ragged kernel over the
    same left-padded buffer (what runs without the stamp).  GB/s counts the
    bytes the cascade must read: the prefix once plus every row's private
    keys and values.  Each timed call follows a 1 GiB write (4x the MALL),
    so both kernels read their bytes from HBM; medians over `iters` calls."""
    import numpy as np
    B, Hq, Hkv, D, P, sp = 8, 32, 8, 128, 16384, 512
    pads = [0, 64, 128, 32, 5, 0, 17, 3]
    L = max(pads) + P + sp
    gen = torch.Generator(device="cuda").manual_seed(1)
    kb = torch.randn(B, Hkv, L, D, generator=gen, device="cuda", dtype=torch.float32).half()
    vb = torch.randn(B, Hkv, L, D, generator=gen, device="cuda", dtype=torch.float32).half()
    for b in range(1, B):  # every row holds row 0's copy of the prefix
        kb[b, :, pads[b]:pads[b] + P] = kb[0, :, pads[0]:pads[0] + P]
        vb[b, :, pads[b]:pads[b] + P] = vb[0, :, pads[0]:pads[0] + P]
    q = torch.randn(B, Hq, 1, D, generator=gen, device="cuda", dtype=torch.float32).half()
    scale = 1.0 / math.sqrt(D)
    c0 = min(pads) + P
    starts = torch.tensor([p + P - c0 for p in pads], dtype=torch.int32, device="cuda")
    l0 = pads[0]
    casc = lambda: ops.sdpa_decode_gqa_cascade(  # noqa: E731
        q, kb[0:1, :, l0:l0 + P], vb[0:1, :, l0:l0 + P], kb[:, :, c0:], vb[:, :, c0:], scale, starts=starts)
    rag = lambda: ops.ragged_decode_attention(q, kb, vb, pads, scale)  # noqa: E731

    flush = mall_flush(torch)
    out = casc()
    qc = quantiles(timed_calls(torch, casc, iters, flush))
    qr = quantiles(timed_calls(torch, rag, iters, flush))
    ms_c, ms_r = qc["median_ms"], qr["median_ms"]
    tok_bytes = Hkv * D * 2 * 2
    need = P * tok_bytes + sum(L - c0 - int(s) for s in starts.tolist()) * tok_bytes
    # spot-check two (row, head) pairs against fp64 over the row's keys
    chk = 0.0
    for b, hq in ((0, 0), (B - 1, Hq - 1)):
        h = hq // (Hq // Hkv)
        kr = kb[b, h, pads[b]:].double().cpu().numpy()
        vr = vb[b, h, pads[b]:].double().cpu().numpy()
        sc = kr @ q[b, hq, 0].double().cpu().numpy() * scale
        pr = np.exp(sc - sc.max())
        ref = pr @ vr / pr.sum()
        got = out[b, hq, 0].double().cpu().numpy()
        chk = max(chk, float(np.abs(got - ref).max() / np.abs(ref).max()))
    del kb, vb
    return {
        "workload": "cascade: B=8 sequences sharing a 16384-token prefix + 512 private tokens (pads 0..128), "
                    "qL 1, 32q/8kv heads, D=128, fp16",
        "ms": round(ms_c, 4),
        "timing": qc,
        "mall": "1 GiB write before every timed call (cold MALL for both kernels)",
        "gbs": round(need / ms_c / 1e6, 1),
        "frac_hbm": round(need / ms_c / 1e6 / HBM_PEAK_GBS, 4),
        "bytes_read_once": need,
        "ragged_same_buffer_ms": round(ms_r, 4),
        "ragged_timing": qr,
        "speedup_vs_ragged": round(ms_r / ms_c, 2),
        "max_rel_spot": chk,
    }


# ------------------------------------------------------------------- MoE

MOE_CONFIGS = {
    # name: (experts, hidden, expert intermediate, top-k, tokens, gate/up codec, down codec)
    "C4": (128, 2048, 768, 8, 32, "q4_k", "q6_k"),
    "C5": (256, 7168, 2048, 8, 8, "iq2_xxs", "iq2_xxs"),
}
BLOCK_BYTES = {"q4_k": 144, "q6_k": 210, "iq2_xxs": 66}


def bench_moe(torch, ops, which, iters=50):
    """Workloads C4 and C5: one MoE decode layer (router top-k, fused
    gate|up GLU gather writing h in the activation dtype, down gather with
    the routing mix folded in) over
    the tokens' ragged per-expert segments.  Router logits and x are numpy
    default_rng(0) draws; weights are N(0, 0.02) drawn on the GPU (torch
    generator, seed 0) and quantised by kq_quantize -- every expert for C4,
    the experts the router touches for C5 (the others hold zero blocks and
    are never read).  C4 rotates two copies of the expert stacks (783 MB,
    > 2x the 256 MB MALL); C5's touched experts alone exceed it.  After
    timing, four tokens' outputs are checked against fp64 over the library's
    bit-exact dequantization of the same wire bytes."""
    import numpy as np
    E, H, I, topk, T, cgu, cd = MOE_CONFIGS[which]
    rng = np.random.default_rng(0)
    logits = torch.from_numpy(rng.normal(0.0, 1.0, size=(T, E)).astype(np.float32)).cuda()
    x = torch.from_numpy(rng.normal(0.0, 1.0, size=(T, H)).astype(np.float16)).cuda()
    gen = torch.Generator(device="cuda").manual_seed(0)
    idx0, _ = ops.moe_router_topk(logits, topk, shared_gate=False)
    touched = sorted(set(idx0.cpu().numpy().reshape(-1).tolist()))

    def stack(N, K, codec):
        nb, bpb = K // 256, BLOCK_BYTES[codec]
        out = torch.zeros((E, N, nb * bpb), dtype=torch.uint8, device="cuda")
        experts = range(E) if codec != "iq2_xxs" else touched
        per = max(1, (64 << 20) // (N * K * 4))  # quantise ~64 MB of fp32 at a time
        ex = list(experts)
        for i in range(0, len(ex), per):
            chunk = ex[i:i + per]
            w = torch.randn((len(chunk) * N, K), generator=gen, device="cuda") * 0.02
            q = ops.quantize(w, codec)[0].view(len(chunk), N, nb * bpb)
            for j, e in enumerate(chunk):
                out[e].copy_(q[j])
            del w, q
        return out

    copies = 2 if which == "C4" else 1
    sets = [(stack(I, H, cgu), stack(I, H, cgu), stack(H, I, cd)) for _ in range(copies)]

    # h in the activation dtype (fp16): the down gather reads it as it is
    def step(g, u, d):
        idx, sc = ops.moe_router_topk(logits, topk, shared_gate=False)
        h = ops.moe_glu_gather_kq(x, g, u, cgu, idx, out_dtype=x.dtype)
        return ops.gather_qmv_mix_ns_kq(h, d, cd, idx, sc)

    g, outs = capture(torch, lambda: [step(*st) for st in sets])
    ms = time_graph(torch, g, iters, 3) / copies
    qm = quantiles([t / copies for t in replay_samples(torch, g, iters)])
    del g
    idx, sc = ops.moe_router_topk(logits, topk, shared_gate=False)
    uniq = int(torch.unique(idx).numel())
    per_expert = 2 * I * (H // 256) * BLOCK_BYTES[cgu] + H * (I // 256) * BLOCK_BYTES[cd]
    act_bytes = T * H * 2 + 2 * T * topk * I * x.element_size() + T * topk * H * 4 * 2 + T * H * 4
    byts = uniq * per_expert + act_bytes
    # spot check: tokens 0, 1, T/2, T-1 of the first copy against fp64
    y = outs[0].cpu().numpy()
    ids, w = idx.cpu().numpy(), sc.cpu().numpy().astype(np.float64)
    xf = x.cpu().numpy().astype(np.float64)
    gs, us, ds = sets[0]
    deq = {}
    worst = 0.0
    for t in sorted({0, 1, T // 2, T - 1}):
        ref = np.zeros(H)
        for s_, e in enumerate(ids[t]):
            if e not in deq:
                deq[e] = tuple(ops.dequantize(m[e], None, c).double().cpu().numpy()
                               for m, c in ((gs, cgu), (us, cgu), (ds, cd)))
            G, U, Dn = deq[e]
            gv, uv = G @ xf[t], U @ xf[t]
            ref += w[t, s_] * (Dn @ (gv / (1.0 + np.exp(-gv)) * uv))
        worst = max(worst, float(np.abs(y[t] - ref).max() / max(np.abs(ref).max(), 1e-30)))
    del sets, outs
    torch.cuda.empty_cache()
    return {
        "workload": f"{which} MoE decode layer: {E} experts, hidden {H}, expert intermediate {I}, top-{topk}, "
                    f"{T} tokens, gate/up {cgu}, down {cd}",
        "unique_experts": uniq, "ms": round(ms, 4), "timing_per_layer": qm, "algorithmic_bytes": byts,
        "gbs": round(byts / ms / 1e6, 1), "frac_hbm": round(byts / ms / 1e6 / HBM_PEAK_GBS, 4),
        "tokens_per_s": round(T / ms * 1e3, 1), "max_rel_spot": worst,
    }


# -------------------------------------------------------------- CPU baseline

def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(layer_wires, B, budget_s=12.0, numpy_budget_s=8.0):
    """The CPU figures beside the C2 line, on one C2 layer (7 matrices,
    122.6 MB of wire) at B rows:
      value: the oracle's OpenMP dequant-fused fp32 matmul (oracle/kq_oracle.c
             kqo_qmm_f32), repeated until ~budget_s, on the host threads this
             process may use (the affinity set, capped by OMP_NUM_THREADS: the
             GPU box grants one GPU's CPU share);
      numpy: numpy's vectorised dequantization (oracle/kquant.py) to fp32,
             then x @ W^T through numpy's BLAS, matrix by matrix until
             ~numpy_budget_s.
    layer_wires: {name: uint8 numpy wire} of one layer."""
    import numpy as np
    from oracle import kquant as okq
    rng = np.random.default_rng(1)
    layer = [(layer_wires[name], N, K, codec) for name, N, K, codec in LAYER]
    xs = {K: rng.normal(0, 1, size=(B, K)).astype(np.float16) for K in (HIDDEN, INTER)}
    affinity = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "").strip()
    nthreads = min(affinity, int(omp)) if omp.isdigit() and int(omp) > 0 else affinity
    done, t0 = 0, time.perf_counter()
    while True:
        for wire, _, K, codec in layer:
            okq.qmm_f32_cpu(xs[K], wire, codec, nthreads=nthreads)
        done += 1
        el = time.perf_counter() - t0
        if el >= budget_s or done >= 50:
            break
    gbs = done * layer_bytes(B) / el / 1e9
    # numpy dequant + BLAS, one matrix at a time, smallest first, until the
    # budget (at least one matrix: the numpy path covers only part of a layer
    # within the budget)
    deq = {"q4_k": okq.dequant_q4_k_np, "q6_k": okq.dequant_q6_k_np, "iq2_xxs": okq.dequant_iq2_xxs_np}
    order = sorted(layer, key=lambda m: m[0].nbytes)
    nbytes, mats, t1 = 0, 0, time.perf_counter()
    while True:
        wire, N, K, codec = order[mats % len(order)]
        w = deq[codec](wire).reshape(N, K)
        _ = xs[K].astype(np.float32) @ w.T
        nbytes += wire.nbytes
        mats += 1
        el_np = time.perf_counter() - t1
        if el_np >= numpy_budget_s:
            break
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": nthreads, "kind": "port",
            "sample": f"{done} pass(es) of one C2 layer (7 matrices, 122.6 MB of wire) at B={B}, "
                      f"{el:.1f} s, oracle/kq_oracle.c kqo_qmm_f32 (OpenMP, fp32)",
            "cpu_model": _cpu_model(), "host_threads_available": affinity,
            "numpy_blas": {"value": round(nbytes / el_np / 1e9, 4), "unit": "GB/s",
                           "sample": f"{mats} of the layer's matrices, smallest first ({nbytes / 1e6:.1f} MB of "
                                     f"wire), numpy dequantization to fp32 then x @ W^T (numpy BLAS), "
                                     f"{el_np:.1f} s"}}


# ------------------------------------------------------------ HBM traffic

COPY_BYTES = 256 << 20


def pmc_pass(args):
    """Body of one rocprofv3 --pmc child run: a few steps of the same
    launches over a 4-layer stack, then one plain 256 MiB device copy whose
    counter value calibrates the counter."""
    import torch
    from gmlx_amd import ops
    stack, rng = make_stack(torch, ops, 4)
    x, xd = make_inputs(torch, rng, args.batch)
    for _ in range(3):
        step_fn(ops, stack, x, xd)
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print("pmc pass done", flush=True)


def measure_traffic(batch, timeout=240):
    """HBM bytes per launch of each kernel from two rocprofv3 --pmc runs
    (FETCH_SIZE, WRITE_SIZE; KiB per dispatch), each scaled by what the same
    counter reads for the 256 MiB copy.  Runs before this process touches
    the GPU.  Returns {kernel: {"fetch": B, "write": B}} or None."""
    import csv
    import glob
    import shutil
    import subprocess
    import tempfile
    if shutil.which("rocprofv3") is None:
        return None
    out = {}
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        d = tempfile.mkdtemp(prefix="kq_pmc_")
        cmd = ["rocprofv3", "--pmc", ctr, "--output-format", "csv", "-d", d, "-o", "pmc", "--",
               sys.executable, os.path.abspath(__file__), "--pmc-pass", "--batch", str(batch)]
        try:
            r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
        except subprocess.TimeoutExpired:
            shutil.rmtree(d, ignore_errors=True)
            return None
        files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
        if r.returncode != 0 or not files:
            shutil.rmtree(d, ignore_errors=True)
            return None
        per = {}
        copy_kib = []
        for row in csv.DictReader(open(files[0])):
            name, v = row.get("Kernel_Name", ""), float(row["Counter_Value"])
            if "copyBuffer" in name or "copy" in name.lower() and int(row.get("Grid_Size", "0")) >= COPY_BYTES // 64:
                copy_kib.append(v)
            for k in KERNEL_FAMILIES:
                if k in name:
                    per.setdefault(k, []).append(v)
        shutil.rmtree(d, ignore_errors=True)
        if not copy_kib:
            return None
        # the copy reads and writes COPY_BYTES once each
        scale = COPY_BYTES / (max(copy_kib) * 1024.0)
        for k, vals in per.items():
            out.setdefault(k, {})["fetch" if ctr == "FETCH_SIZE" else "write"] = \
                sum(vals) / len(vals) * 1024.0 * scale
            out[k]["scale_" + ctr.lower()] = round(scale, 4)
    return out


# --------------------------------------------------------------------- main

def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-sdpa", action="store_true")
    ap.add_argument("--no-cascade", action="store_true")
    ap.add_argument("--no-moe", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-traffic", action="store_true", help="skip the two rocprofv3 --pmc passes")
    ap.add_argument("--pmc-pass", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.pmc_pass:
        return pmc_pass(args)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    # HBM traffic counters come from child processes started before this
    # process touches the GPU
    traffic = None if args.no_traffic else measure_traffic(args.batch)
    if traffic is not None:
        log(f"[bench] pmc traffic per launch: { {k: {kk: round(vv) for kk, vv in v.items()} for k, v in traffic.items()} }")

    import torch
    from gmlx_amd import ops
    import gmlx_amd
    gmlx_amd.lib()  # fails loudly when the HIP library is missing
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)

    log(f"[bench] building {args.layers}-layer Q4_K_M stack on {torch.cuda.get_device_name(0)}")
    stack, rng = make_stack(torch, ops, args.layers)
    B = args.batch
    x, xd = make_inputs(torch, rng, B)
    g, outs = capture(torch, lambda: step_fn(ops, stack, x, xd))
    # graph replays must reproduce the eager result bit for bit
    g.replay()
    torch.cuda.synchronize()
    eager = step_fn(ops, stack, x, xd)
    torch.cuda.synchronize()
    replay_ok = all(torch.equal(a, b) for a, b in zip(outs, eager))
    log(f"[bench] graph captured, replay==eager: {replay_ok}")

    torch.cuda.synchronize()
    ms = time_graph(torch, g, args.steps, args.warmup)
    step_bytes = args.layers * layer_bytes(B)
    value = step_bytes / ms / 1e6
    launches = 4 * args.layers
    # per-replay distribution (outside the contract's timed region)
    step_q = quantiles(replay_samples(torch, g, max(50, args.steps)))
    log(f"[bench] B={B}: {ms:.3f} ms/step, {value:.1f} GB/s (replays: median {step_q['median_ms']:.3f}, "
        f"p10 {step_q['p10_ms']:.3f}, p90 {step_q['p90_ms']:.3f} ms)")
    del g
    spot = spot_check_layer(torch, ops, stack[0], x, xd)
    log(f"[bench] max_rel_spot per launch (layer 0 vs fp64): {spot}")
    copyp = copy_peak(torch)
    log(f"[bench] copy peak: {copyp['gbs_median']} GB/s ({copyp['frac_of_8tbs']} of 8 TB/s)")

    # per-kernel launch durations: each kernel's launches of the step, alone
    # in a graph, timed with HIP events on the replay stream
    kernels = {}
    for launch, _ in LAUNCHES:
        kernels.setdefault(family(kernel_of(launch, B)), []).append(launch)
    per_kernel = {}
    for kname, lset in kernels.items():
        gk, _ = capture(torch, lambda: step_fn(ops, stack, x, xd, only=set(lset)))
        msk = time_graph(torch, gk, args.steps, args.warmup)
        n = args.layers * len(lset)
        byts = args.layers * sum(launch_bytes(l, B) for l in lset)
        per_kernel[kname] = {"launches": lset, "instances": sorted({kernel_of(l, B) for l in lset}),
                             "launches_per_step": n, "avg_launch_us": round(msk * 1e3 / n, 3),
                             "bytes_per_launch": byts // n, "gbs": round(byts / msk / 1e6, 1)}
        log(f"[bench] {kname} ({'+'.join(lset)}): {msk * 1e3 / n:.2f} us/launch, {byts / msk / 1e6:.1f} GB/s")
        del gk
    dominant = max(per_kernel, key=lambda k: per_kernel[k]["avg_launch_us"] * per_kernel[k]["launches_per_step"])
    # and each launch of a layer alone
    per_launch = {}
    for launch, _ in LAUNCHES:
        gl, _ = capture(torch, lambda: step_fn(ops, stack, x, xd, only={launch}))
        msl = time_graph(torch, gl, args.steps, args.warmup)
        byts = args.layers * launch_bytes(launch, B)
        per_launch[launch] = {"kernel": kernel_of(launch, B), "avg_us": round(msl * 1e3 / args.layers, 3),
                              "bytes": launch_bytes(launch, B), "gbs": round(byts / msl / 1e6, 1),
                              "max_rel_spot": spot[launch]}
        log(f"[bench]   {launch}: {msl * 1e3 / args.layers:.2f} us, {byts / msl / 1e6:.1f} GB/s")
        del gl

    # the fused MLP (kq_fused_mlp: gmlx's _FusedMLP, gate|up -> SwiGLU -> down
    # in one launch, down reading the h it produced) against the two split
    # launches on independent inputs, 36 layers each, graph replay
    mlp = None
    if B <= 8:
        def split_mlp():
            return step_fn(ops, stack, x, xd, only={"gate_up", "down"})

        def fused_mlp():
            return [ops.fused_mlp(x, L["gate"], L["up"], L["down"], "q4_k", "q6_k") for L in stack]
        mlp = {}
        for name, fn in (("split_us", split_mlp), ("fused_us", fused_mlp)):
            gm, _ = capture(torch, fn)
            mlp[name] = round(quantiles(replay_samples(torch, gm, max(50, args.steps)))["median_ms"] * 1e3
                              / args.layers, 3)
            del gm
        mlp["fused_single_launch"] = ops.counts()["fused_mlp_launches"] > 0
        log(f"[bench] MLP per layer: split gate|up + down {mlp['split_us']} us, fused {mlp['fused_us']} us")

    per_batch = {}
    if not args.no_sweep:
        for b in (1, 2, 4, 8, 16, 32, 64):
            xb, xdb = make_inputs(torch, rng, b)
            gb, _ = capture(torch, lambda: step_fn(ops, stack, xb, xdb))
            time_graph(torch, gb, 3, 2)
            qb = quantiles(replay_samples(torch, gb, 50))
            msb = qb["median_ms"]
            gbs = args.layers * layer_bytes(b) / msb / 1e6
            per_batch[str(b)] = {"ms_per_step": round(msb, 4), "timing": qb, "gbs": round(gbs, 1),
                                 "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                                 "tflops": round(2 * b * args.layers * sum(N * K for _, N, K, _ in LAYER)
                                                 / msb / 1e9, 2)}
            log(f"[bench] sweep B={b}: {msb:.3f} ms/step, {gbs:.1f} GB/s")
            del gb

    moe = None
    if not args.no_moe:
        moe = {}
        for which in MOE_CONFIGS:
            moe[which] = bench_moe(torch, ops, which)
            log(f"[bench] moe {which}: {moe[which]['ms']} ms, {moe[which]['gbs']} GB/s over "
                f"{moe[which]['unique_experts']} touched experts")

    sdpa = None
    if not args.no_sdpa:
        sdpa = bench_sdpa(torch, ops, cpu=not args.no_cpu)
        log(f"[bench] sdpa C3: {sdpa['ms']} ms, {sdpa['kv_gbs']} GB/s, {sdpa['kv_tokens_per_s']:.3e} tok/s; "
            f"8-bit KV {sdpa['q8_kv']['ms']} ms, {sdpa['q8_kv']['kv_gbs']} GB/s, "
            f"{sdpa['q8_kv']['kv_tokens_per_s']:.3e} tok/s")
        if sdpa["cpu_baseline"]:
            log(f"[bench] sdpa C3 cpu baseline: {sdpa['cpu_baseline']['kv_gbs']} GB/s, "
                f"{sdpa['cpu_baseline']['kv_tokens_per_s']:.3e} tok/s on {sdpa['cpu_baseline']['cores']} threads")

    cascade = None
    if not args.no_cascade:
        cascade = bench_cascade(torch, ops)
        log(f"[bench] cascade: {cascade['ms']} ms, {cascade['gbs']} GB/s on bytes read once, "
            f"{cascade['speedup_vs_ragged']}x the ragged kernel on the same buffer")

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline({k: v.cpu().numpy() for k, v in stack[0].items()}, B)
        log(f"[bench] cpu baseline: {cpu['value']} GB/s on {cpu['cores']} threads ({cpu['cpu_model']}); "
            f"numpy dequant + BLAS {cpu['numpy_blas']['value']} GB/s")

    dk = per_kernel[dominant]
    achieved = dk["bytes_per_launch"] / dk["avg_launch_us"] / 1e3
    tr = None
    if traffic is not None:
        if dominant in traffic and "fetch" in traffic[dominant] and "write" in traffic[dominant]:
            tr = round(traffic[dominant]["fetch"] + traffic[dominant]["write"])
    res = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "step_replays": step_q,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": f"C2 Qwen3-8B Q4_K_M linear stack: {args.layers} layers x "
                               "(q|k|v, o, gate|up, down), distinct weights per layer",
                   "batch": B, "layers": args.layers, "hidden": HIDDEN, "intermediate": INTER,
                   "weights_per_step_bytes": args.layers * sum(wire_bytes(N, K, c) for _, N, K, c in LAYER),
                   "launches_per_step": launches, "graph_replay_equals_eager": replay_ok},
        "roofline": {"bound": "hbm", "kernel": dominant,
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": tr,
                     "algorithmic_bytes_per_launch": dk["bytes_per_launch"],
                     "avg_launch_us": dk["avg_launch_us"]},
        "copy_peak": copyp,
        "kernels": per_kernel,
        "launches": per_launch,
        "mlp": mlp,
        "traffic_per_launch": traffic,
        "cpu_baseline": cpu,
        "per_batch": per_batch,
        "sdpa": sdpa,
        "cascade": cascade,
        "moe": moe,
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
