"""Dequant-fused quantized matmul parity (kq_quantized_matmul_grouped through
the C ABI): max-rel <= 2e-3 against the fp64 oracle, plus the reference's
structural properties (row independence of concatenated wires,
gmlx/occupancy_fuse.py:32-34; B=1 inside a batch equals M=1,
tests/test_batch_parity.py:147-159; permutation; determinism)."""
import os

import numpy as np
import pytest

from helpers import BF16_TOL, TOL, fp16_rows, quantized_weights
from oracle import kquant as okq

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _mm(x16, wire, codec, **kw):
    from gmlx_amd import ops
    return ops.quantized_matmul(_dev(x16), _dev(wire), None, codec, **kw)


def test_config1_q4k_matvec():
    """Workload C1: Q4_K 3072x1024 from N(0, 0.02), x fp16 [1, 1024] N(0, 1), seed 0."""
    rng = np.random.default_rng(0)
    w = rng.normal(0.0, 0.02, size=(3072, 1024)).astype(np.float32)
    wire = okq.quantize(w, "q4_k")
    x = rng.normal(0.0, 1.0, size=(1, 1024)).astype(np.float16)
    ref = okq.qmm_ref(x, wire, "q4_k")
    got = _mm(x, wire, "q4_k").float().cpu().numpy()
    assert got.shape == (1, 3072)
    assert okq.max_rel(got, ref) <= TOL


@pytest.mark.parametrize("codec", ["q4_k", "q6_k", "iq2_xxs"])
@pytest.mark.parametrize("M", [1, 2, 3, 5, 8, 13, 16, 17, 31, 33, 64, 65])
def test_small_m_parity(codec, M):
    rng = np.random.default_rng(100 + M)
    N, K = 200, 1280                # N not a multiple of 16, K = 5 blocks (partial 4-block step)
    wire = quantized_weights(rng, codec, N, K) if codec != "iq2_xxs" else okq.random_valid_blocks(
        rng, codec, N * K // 256).reshape(N, -1)
    x = fp16_rows(rng, M, K)
    ref = okq.qmm_ref(x, wire, codec)
    got = _mm(x, wire, codec).float().cpu().numpy()
    assert okq.max_rel(got, ref) <= TOL, okq.max_rel(got, ref)


@pytest.mark.parametrize("codec", ["q4_k", "q6_k"])
def test_config2_shapes_b8(codec):
    """Config 2 geometry (K 4096 and 12288) at B=8."""
    rng = np.random.default_rng(7)
    for N, K in [(1024, 4096), (512, 12288)]:
        wire = quantized_weights(rng, codec, N, K)
        x = fp16_rows(rng, 8, K)
        ref = okq.qmm_ref(x, wire, codec)
        got = _mm(x, wire, codec).float().cpu().numpy()
        assert okq.max_rel(got, ref) <= TOL


@pytest.mark.parametrize("M", [1, 8, 16])
def test_config2_qkv_group(M, monkeypatch):
    """The q|k|v group of a Qwen3-8B Q4_K_M layer (Q4_K q, k with Q6_K v) on
    default routing (the one-shot kernel at 1 and 8 rows, two K slices on the
    streaming kernel at 16) matches the fp64 reference, repeats bitwise,
    agrees with the LDS-staged path and leaves the workspace's arrival
    counters zero."""
    import torch
    from gmlx_amd import _lib, ops
    for k in PATH_KNOBS:
        monkeypatch.delenv(k, raising=False)
    rng = np.random.default_rng(30 + M)
    K = 4096
    mats = [(quantized_weights(rng, "q4_k", 4096, K), "q4_k"), (quantized_weights(rng, "q4_k", 1024, K), "q4_k"),
            (quantized_weights(rng, "q6_k", 1024, K), "q6_k")]
    x16 = fp16_rows(rng, M, K)
    x = _dev(x16)
    items = [(x, _dev(w), c) for w, c in mats]
    outs = [ops.quantized_matmul_grouped(items, out_dtype=torch.float32) for _ in range(2)]
    torch.cuda.synchronize()
    for (w, c), o, o2 in zip(mats, outs[0], outs[1]):
        assert okq.max_rel(o.cpu().numpy(), okq.qmm_ref(x16, w, c)) <= TOL, c
        assert torch.equal(o, o2)
    ws = ops._WS.get("matmul", x.device, ops._stream(x).value, 0)
    assert int(ws[:_lib.MATMUL_COUNTER_BYTES].count_nonzero()) == 0
    monkeypatch.setenv("GMLX_KQ_STREAM", "0")
    staged = ops.quantized_matmul_grouped(items, out_dtype=torch.float32)
    for o, o2 in zip(outs[0], staged):
        assert okq.max_rel(o.cpu().numpy(), o2.cpu().numpy()) <= TOL


def test_bf16_activations_and_f32_out():
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(8)
    wire = quantized_weights(rng, "q4_k", 96, 512)
    x32 = rng.normal(0, 1, size=(4, 512)).astype(np.float32)
    xb = torch.from_numpy(x32).to(torch.bfloat16)
    ref = okq.qmm_ref(xb.float().numpy(), wire, "q4_k")
    got = ops.quantized_matmul(xb.cuda(), _dev(wire), None, "q4_k").float().cpu().numpy()
    # a bf16 output carries 8 mantissa bits: its rounding alone is up to 2^-9 relative
    assert okq.max_rel(got, ref) <= BF16_TOL
    got32 = ops.quantized_matmul(xb.cuda(), _dev(wire), None, "q4_k", out_dtype=torch.float32)
    assert got32.dtype == torch.float32
    assert okq.max_rel(got32.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("path", [{"GMLX_KQ_STREAM": "0", "GMLX_KQ_MV": "0"},
                                  {"GMLX_KQ_STREAM": "0", "GMLX_KQ_MV": "2"}, {}])
def test_grouped_equals_separate_bitwise(path, monkeypatch):
    """q|k|v with mixed codecs in one launch == three separate launches:
    bitwise when both take the same kernel (the general or the LDS-staged
    path forced), within tolerance under the default routing (a mixed-codec
    group and a single matrix may take different kernels, whose k-order
    differs)."""
    from gmlx_amd import ops
    for k, v in path.items():
        monkeypatch.setenv(k, v)
    rng = np.random.default_rng(9)
    K = 1024
    wq = quantized_weights(rng, "q4_k", 256, K)
    wk = quantized_weights(rng, "q4_k", 64, K)
    wv = quantized_weights(rng, "q6_k", 64, K)
    x16 = fp16_rows(rng, 4, K)
    x = _dev(x16)
    outs = ops.quantized_matmul_grouped([(x, _dev(wq), "q4_k"), (x, _dev(wk), "q4_k"), (x, _dev(wv), "q6_k")])
    for o, (w, c) in zip(outs, [(wq, "q4_k"), (wk, "q4_k"), (wv, "q6_k")]):
        sep = ops.quantized_matmul(x, _dev(w), None, c)
        if path:
            assert np.array_equal(o.cpu().numpy().view(np.uint16), sep.cpu().numpy().view(np.uint16))
        else:
            ref = okq.qmm_ref(x16, w, c)
            assert okq.max_rel(o.float().cpu().numpy(), ref) <= TOL
            assert okq.max_rel(sep.float().cpu().numpy(), ref) <= TOL


def test_row_concatenated_wire_is_row_independent():
    """Output rows of a row-concatenated wire equal the separate matmuls."""
    rng = np.random.default_rng(10)
    K = 512
    wa = quantized_weights(rng, "q4_k", 48, K)
    wb = quantized_weights(rng, "q4_k", 80, K)
    x = fp16_rows(rng, 3, K)
    cat = _mm(x, np.concatenate([wa, wb]), "q4_k").cpu().numpy()
    a = _mm(x, wa, "q4_k").cpu().numpy()
    b = _mm(x, wb, "q4_k").cpu().numpy()
    # k-splitting depends on N, so compare within tolerance and exactly when plans agree
    ref = okq.qmm_ref(x, np.concatenate([wa, wb]), "q4_k")
    assert okq.max_rel(cat.astype(np.float32), ref) <= TOL
    assert okq.max_rel(np.concatenate([a, b], axis=1).astype(np.float32), ref) <= TOL


def test_batch_row_equals_single_row_and_permutation():
    rng = np.random.default_rng(12)
    wire = quantized_weights(rng, "q4_k", 160, 2048)
    x = fp16_rows(rng, 8, 2048)
    full = _mm(x, wire, "q4_k").cpu().numpy()
    one = _mm(x[3:4], wire, "q4_k").cpu().numpy()
    assert np.array_equal(full[3:4].view(np.uint16), one.view(np.uint16))
    perm = rng.permutation(8)
    pm = _mm(x[perm], wire, "q4_k").cpu().numpy()
    assert np.array_equal(pm.view(np.uint16), full[perm].view(np.uint16))


def test_deterministic_split_k():
    rng = np.random.default_rng(13)
    wire = quantized_weights(rng, "q6_k", 64, 4096)   # few tiles -> k split across waves
    x = fp16_rows(rng, 5, 4096)
    outs = [_mm(x, wire, "q6_k").cpu().numpy() for _ in range(4)]
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint16), outs[0].view(np.uint16))
    ref = okq.qmm_ref(x, wire, "q6_k")
    assert okq.max_rel(outs[0].astype(np.float32), ref) <= TOL


def test_graph_keeps_its_workspace_when_a_later_capture_grows_it():
    """A split launch (K = 12288 at 8 rows: partial tiles and arrival
    counters in the workspace) captured in graph A; then graph B, captured
    on the same capture stream, needs a larger workspace of the same family,
    which replaces the stream's buffer.  A still holds the buffer it was
    captured with (kept alive, counters left zero), so its replays, between
    B's replays and eager calls, equal the eager result bitwise."""
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(17)
    w_small = _dev(quantized_weights(rng, "q6_k", 256, 12288))
    w_big = _dev(quantized_weights(rng, "q6_k", 4096, 12288))
    x = _dev(fp16_rows(rng, 8, 12288))
    eager = ops.quantized_matmul(x, w_small, None, "q6_k")
    eager_big = ops.quantized_matmul(x, w_big, None, "q6_k")
    torch.cuda.synchronize()
    ga, gb = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(ga):
        out_a = ops.quantized_matmul(x, w_small, None, "q6_k")
    with torch.cuda.graph(gb):
        out_b = ops.quantized_matmul(x, w_big, None, "q6_k")
    torch.cuda.synchronize()
    for _ in range(3):
        ga.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_a, eager)
        gb.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_b, eager_big)
        assert torch.equal(ops.quantized_matmul(x, w_big, None, "q6_k"), eager_big)
    ref = okq.qmm_ref(x.cpu().numpy(), w_big.cpu().numpy()[:64], "q6_k")
    assert okq.max_rel(eager_big[:, :64].float().cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("wgs", ["1", "3"])
def test_stream_multi_round_wide_range_rows(wgs, monkeypatch):
    """Q4_K streaming launches on 1 and 3 workgroups (every workgroup walks
    many rounds of tiles through the ring) with bf16 rows of very different
    magnitudes (per-row exponents: the sums and the minimum term at large
    scales): every row matches the fp64 reference on its own scale."""
    import torch
    from gmlx_amd import ops
    monkeypatch.setenv("GMLX_KQ_STREAM", "2")
    monkeypatch.setenv("GMLX_KQ_STREAM_WGS", wgs)
    rng = np.random.default_rng(23)
    N, K, M = 1000, 4096, 6
    wire = quantized_weights(rng, "q4_k", N, K)
    x = rng.normal(0.0, 1.0, size=(M, K)).astype(np.float32)
    x[0] *= 3e4
    x[1] = np.abs(x[1]) * 5e3 + 2e3
    x[2] *= 1e-5
    xd = torch.from_numpy(x).to(torch.bfloat16)
    ref = okq.qmm_ref(xd.float().numpy(), wire, "q4_k")
    got = ops.quantized_matmul(xd.cuda(), _dev(wire), None, "q4_k", out_dtype=torch.float32).cpu().numpy()
    for m in range(M):
        assert okq.max_rel(got[m], ref[m]) <= TOL, (m, okq.max_rel(got[m], ref[m]))


@pytest.mark.parametrize("nb", [1, 2, 3, 4, 5, 8, 16, 17, 48])
def test_k_block_counts(nb):
    """Every K split shape of the 4-wave workgroup: waves with no step,
    partial last steps, several steps per wave."""
    rng = np.random.default_rng(14 + nb)
    K = 256 * nb
    for codec in ("q4_k", "q6_k"):
        wire = quantized_weights(rng, codec, 40, K)
        x = fp16_rows(rng, 3, K)
        ref = okq.qmm_ref(x, wire, codec)
        got = _mm(x, wire, codec).float().cpu().numpy()
        assert okq.max_rel(got, ref) <= TOL, (codec, nb)


def test_module_forward():
    import torch
    from gmlx_amd.nn import KQuantLinear
    rng = np.random.default_rng(15)
    wire = quantized_weights(rng, "q4_k", 128, 512)
    mod = KQuantLinear(512, 128, bias=True, codec="q4_k").cuda()
    mod.weight.copy_(_dev(wire))
    with torch.no_grad():
        mod.bias.copy_(torch.linspace(-1, 1, 128))
    x = fp16_rows(rng, 3, 512)
    got = mod(_dev(x).reshape(3, 1, 512)).float().cpu().numpy().reshape(3, 128)
    ref = okq.qmm_ref(x, wire, "q4_k") + np.linspace(-1, 1, 128)
    assert okq.max_rel(got, ref) <= TOL


# The small-batch paths of kq_quantized_matmul_grouped, forced in turn: the
# producer / consumer weight-streaming kernel (M <= 16, K of 2, 4, 6, 8, 12 or
# 16 super-blocks, or K cut into such slices: by default past 16 super-blocks,
# GMLX_KQ_SPLITK=s slices where they divide K), the LDS-staged persistent
# path (kq_mv) and the general tiled path.  Small grids make every workgroup walk many tiles, with partial ring
# rounds.
SMALL_BATCH_PATHS = [
    ("default routing", {}),
    ("stream, 3 workgroups", {"GMLX_KQ_STREAM": "2", "GMLX_KQ_STREAM_WGS": "3"}),
    ("stream, 13 workgroups", {"GMLX_KQ_STREAM": "2", "GMLX_KQ_STREAM_WGS": "13"}),
    ("stream, full grid", {"GMLX_KQ_STREAM": "2"}),
    ("stream, split 2, 5 workgroups", {"GMLX_KQ_STREAM": "2", "GMLX_KQ_SPLITK": "2", "GMLX_KQ_STREAM_WGS": "5"}),
    ("stream, split 3", {"GMLX_KQ_STREAM": "2", "GMLX_KQ_SPLITK": "3"}),
    ("stream, split 4, 13 workgroups", {"GMLX_KQ_STREAM": "2", "GMLX_KQ_SPLITK": "4", "GMLX_KQ_STREAM_WGS": "13"}),
    ("mv, default grid", {"GMLX_KQ_STREAM": "0", "GMLX_KQ_MV": "2"}),
    ("mv, 3 workgroups", {"GMLX_KQ_STREAM": "0", "GMLX_KQ_MV": "2", "GMLX_KQ_MV_WGS": "3"}),
    ("mv, 7 workgroups, ring 2", {"GMLX_KQ_STREAM": "0", "GMLX_KQ_MV": "2", "GMLX_KQ_MV_WGS": "7",
                                  "GMLX_KQ_MV_DEPTH": "2"}),
    ("mv, 5 workgroups, ring 1", {"GMLX_KQ_STREAM": "0", "GMLX_KQ_MV": "2", "GMLX_KQ_MV_WGS": "5",
                                  "GMLX_KQ_MV_DEPTH": "1"}),
    ("general", {"GMLX_KQ_STREAM": "0", "GMLX_KQ_MV": "0"}),
]
PATH_KNOBS = ("GMLX_KQ_STREAM", "GMLX_KQ_STREAM_WGS", "GMLX_KQ_SPLITK", "GMLX_KQ_MV", "GMLX_KQ_MV_WGS",
              "GMLX_KQ_MV_DEPTH")


@pytest.mark.parametrize("codec,N,K,M", [
    ("q4_k", 9000, 4096, 5),       # 563 tiles: several tiles per workgroup, odd count
    ("q4_k", 777, 3328, 16),       # 13 blocks: waves past the last block
    ("q4_k", 300, 12288, 3),       # 48 blocks: three blocks per wave
    ("q6_k", 1040, 4096, 8),
    ("q6_k", 200, 8192, 2),        # 32 blocks: two Q6_K blocks per wave
    ("iq2_xxs", 520, 7168, 3),     # 28 blocks
    ("q4_k", 64, 256, 1),          # single block, single wave
    ("q6_k", 600, 12288, 8),       # x past LDS: last 4096 columns in registers
    ("q4_k", 500, 12288, 6),
    ("q4_k", 300, 8192, 16),       # two blocks per wave, the second from registers
    ("iq2_xxs", 256, 12288, 7),
    ("q4_k", 1000, 1024, 8),       # stream: 63 tiles, a partial last tile
    ("q4_k", 4000, 512, 2),        # stream: 250 tiles, several rounds on small grids
    ("q6_k", 700, 2048, 7),
    ("iq2_xxs", 330, 4096, 4),
    ("q4_k", 333, 1536, 5),        # stream: 6 blocks, 6 consumers
    ("q6_k", 200, 3072, 8),        # stream: 12 blocks, 12 consumers
    ("iq2_xxs", 150, 1536, 3),
    ("q4_k", 2000, 2048, 16),      # stream: 16 rows, one block per consumer, activations in registers
    ("q4_k", 700, 4096, 13),       # stream: 16-row form, two passes of activation staging
    ("q6_k", 500, 4096, 12),
    ("iq2_xxs", 300, 3072, 9),
    ("q4_k", 16, 4096, 5),         # stream: one tile (one workgroup), staged activations
    ("q6_k", 8, 4096, 8),          # stream: one partial tile, staged activations, two ring slots
    ("iq2_xxs", 40, 4096, 2),      # stream: three tiles, the last partial, staged activations
    ("q4_k", 48, 2048, 1),         # stream: 8 blocks per row, overlapping row loads
])
def test_small_batch_paths(codec, N, K, M, monkeypatch):
    """Every small-batch path matches the fp64 reference on the same inputs."""
    rng = np.random.default_rng(N + K + M)
    if codec == "iq2_xxs":
        wire = okq.random_valid_blocks(rng, codec, N * K // 256).reshape(N, -1)
    else:
        wire = quantized_weights(rng, codec, N, K)
    x = fp16_rows(rng, M, K)
    ref = okq.qmm_ref(x, wire, codec)
    for name, env in SMALL_BATCH_PATHS:
        for k in PATH_KNOBS:
            monkeypatch.delenv(k, raising=False)
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        got = _mm(x, wire, codec).float().cpu().numpy()
        assert okq.max_rel(got, ref) <= TOL, (name, okq.max_rel(got, ref))


@pytest.mark.parametrize("codec,N,K,M,x_dtype", [
    ("q6_k", 4096, 12288, 8, "float16"),    # the Qwen3-8B down projection at batch 8
    ("q4_k", 1000, 12288, 1, "bfloat16"),
    ("q6_k", 515, 14336, 5, "float32"),     # 7 slices, a partial last tile
    ("iq2_xxs", 300, 8192, 3, "float16"),   # 4 slices
    ("q4_k", 700, 7168, 6, "float16"),      # 28 blocks: 7 slices of 4
    ("q6_k", 300, 9216, 4, "bfloat16"),     # 36 blocks: 3 slices of 12
    ("q6_k", 1000, 12288, 13, "float16"),   # 16-row partial tiles
    ("q4_k", 260, 12288, 16, "float32"),
])
def test_split_k_stream(codec, N, K, M, x_dtype, monkeypatch):
    """K past 16 super-blocks at <= 16 rows: the K-sliced streaming launch
    matches the fp64 reference and the unsplit LDS-staged path, repeats
    bitwise, and leaves the workspace's arrival counters zero."""
    import torch
    from gmlx_amd import _lib, ops
    for k in PATH_KNOBS:
        monkeypatch.delenv(k, raising=False)
    rng = np.random.default_rng(N + K + M)
    if codec == "iq2_xxs":
        wire = okq.random_valid_blocks(rng, codec, N * K // 256).reshape(N, -1)
    else:
        wire = quantized_weights(rng, codec, N, K)
    x = _dev(fp16_rows(rng, M, K)).to(getattr(torch, x_dtype))
    ref = okq.qmm_ref(x.float().cpu().numpy(), wire, codec)
    w = _dev(wire)
    monkeypatch.setenv("GMLX_KQ_STREAM", "2")
    outs = [ops.quantized_matmul(x, w, codec=codec, out_dtype=torch.float32) for _ in range(3)]
    torch.cuda.synchronize()
    got = outs[0].cpu().numpy()
    assert okq.max_rel(got, ref) <= TOL, okq.max_rel(got, ref)
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    ws = ops._WS.get("matmul", x.device, ops._stream(x).value, 0)
    assert int(ws[:_lib.MATMUL_COUNTER_BYTES].count_nonzero()) == 0
    monkeypatch.setenv("GMLX_KQ_STREAM", "0")
    monkeypatch.setenv("GMLX_KQ_MV", "2")
    unsplit = ops.quantized_matmul(x, w, codec=codec, out_dtype=torch.float32).cpu().numpy()
    assert okq.max_rel(got, unsplit) <= TOL


@pytest.mark.parametrize("codec,K,M,env", [
    ("q4_k", 4096, 8, {}),
    ("q6_k", 2048, 5, {"GMLX_KQ_STREAM_WGS": "7"}),
    ("q6_k", 12288, 8, {"GMLX_KQ_SPLITK": "6", "GMLX_KQ_STREAM_WGS": "12"}),
    ("q4_k", 3072, 16, {"GMLX_KQ_STREAM_WGS": "5"}),
])
def test_stream_row_pitches_and_partial_tiles(codec, K, M, env, monkeypatch):
    """The streaming kernel's producers keep per-lane chunk offsets of full
    tiles for the first problem's row pitch: a group whose second problem has
    wider rows (padding after each row's blocks) and whose first ends in a
    partial tile takes the general offsets where those differ, and both match
    the fp64 reference."""
    import torch
    from gmlx_amd import ops
    for k in PATH_KNOBS:
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("GMLX_KQ_STREAM", "2")
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    rng = np.random.default_rng(K + M)
    Na, Nb = 1000, 704
    wa = quantized_weights(rng, codec, Na, K)
    wb = quantized_weights(rng, codec, Nb, K)
    x16 = fp16_rows(rng, M, K)
    x = _dev(x16)
    wide = torch.zeros(Nb, wb.shape[1] + 48, dtype=torch.uint8)
    wide[:, :wb.shape[1]] = torch.from_numpy(wb)
    wbv = wide.cuda()[:, :wb.shape[1]]
    ya, yb = ops.quantized_matmul_grouped([(x, _dev(wa), codec), (x, wbv, codec)], out_dtype=torch.float32)
    assert okq.max_rel(ya.cpu().numpy(), okq.qmm_ref(x16, wa, codec)) <= TOL
    assert okq.max_rel(yb.cpu().numpy(), okq.qmm_ref(x16, wb, codec)) <= TOL


@pytest.mark.parametrize("K,M", [(4096, 8), (8192, 3), (1280, 16), (2048, 1)])
def test_mixed_codec_group_paths(K, M, monkeypatch):
    """q|k (Q4_K) with v (Q6_K) in one launch: the mixed LDS-staged kernel
    (rings of 1..3 tiles, small grids) and the general path match the fp64
    reference; an IQ2_XXS member routes the group elsewhere."""
    from gmlx_amd import ops
    rng = np.random.default_rng(K + M)
    wq = quantized_weights(rng, "q4_k", 300, K)
    wk = quantized_weights(rng, "q4_k", 70, K)
    wv = quantized_weights(rng, "q6_k", 90, K)
    wi = okq.random_valid_blocks(rng, "iq2_xxs", 40 * K // 256).reshape(40, -1)
    x16 = fp16_rows(rng, M, K)
    x = _dev(x16)
    mats = [(wq, "q4_k"), (wk, "q4_k"), (wv, "q6_k")]
    refs = [okq.qmm_ref(x16, w, c) for w, c in mats]
    ref_i = okq.qmm_ref(x16, wi, "iq2_xxs")
    for name, env in SMALL_BATCH_PATHS:
        for k in PATH_KNOBS:
            monkeypatch.delenv(k, raising=False)
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        outs = ops.quantized_matmul_grouped([(x, _dev(w), c) for w, c in mats])
        for o, ref in zip(outs, refs):
            assert okq.max_rel(o.float().cpu().numpy(), ref) <= TOL, name
        outs = ops.quantized_matmul_grouped([(x, _dev(w), c) for w, c in mats] + [(x, _dev(wi), "iq2_xxs")])
        for o, ref in zip(outs, refs + [ref_i]):
            assert okq.max_rel(o.float().cpu().numpy(), ref) <= TOL, (name, "with iq2_xxs")


@pytest.mark.parametrize("y_dtype", ["float32", "bfloat16"])
def test_small_batch_output_dtypes(y_dtype, monkeypatch):
    """bf16 activations and f32 / bf16 outputs through the LDS-staged path."""
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(31)
    N, K, M = 333, 2048, 6
    wire = quantized_weights(rng, "q4_k", N, K)
    x32 = rng.normal(0.0, 1.0, size=(M, K)).astype(np.float32)
    xb = torch.from_numpy(x32).to(torch.bfloat16)
    ref = okq.qmm_ref(xb.float().numpy(), wire, "q4_k")
    monkeypatch.setenv("GMLX_KQ_MV", "2")
    monkeypatch.setenv("GMLX_KQ_MV_WGS", "5")
    out, = ops.quantized_matmul_grouped([(xb.cuda(), _dev(wire), "q4_k")], out_dtype=getattr(torch, y_dtype))
    assert out.dtype == getattr(torch, y_dtype)
    assert okq.max_rel(out.float().cpu().numpy(), ref) <= BF16_TOL


@pytest.mark.parametrize("mv", ["stream", "2", "0"])
def test_mixed_codec_group_and_determinism(mv, monkeypatch):
    """q|k (Q4_K) and v (Q6_K) sharing x: one small-batch launch (the
    streaming kernel, the LDS-staged path forced) or the general kernel;
    repeated calls are bitwise identical."""
    from gmlx_amd import ops
    rng = np.random.default_rng(21)
    K = 4096
    wq = quantized_weights(rng, "q4_k", 512, K)
    wk = quantized_weights(rng, "q4_k", 128, K)
    wv = quantized_weights(rng, "q6_k", 128, K)
    x16 = fp16_rows(rng, 8, K)
    x = _dev(x16)
    if mv == "stream":
        monkeypatch.setenv("GMLX_KQ_STREAM", "2")
        monkeypatch.setenv("GMLX_KQ_STREAM_WGS", "4")
    else:
        monkeypatch.setenv("GMLX_KQ_STREAM", "0")
        monkeypatch.setenv("GMLX_KQ_MV_WGS", "4")
        monkeypatch.setenv("GMLX_KQ_MV", mv)
    outs = [ops.quantized_matmul_grouped([(x, _dev(wq), "q4_k"), (x, _dev(wk), "q4_k"), (x, _dev(wv), "q6_k")])
            for _ in range(3)]
    for o in outs[1:]:
        for a, b in zip(o, outs[0]):
            assert np.array_equal(a.cpu().numpy().view(np.uint16), b.cpu().numpy().view(np.uint16))
    for o, (w, c) in zip(outs[0], [(wq, "q4_k"), (wk, "q4_k"), (wv, "q6_k")]):
        assert okq.max_rel(o.float().cpu().numpy(), okq.qmm_ref(x16, w, c)) <= TOL


def test_large_scales_every_route(monkeypatch):
    """Q4_K super-blocks whose sub-block scales reach |d sc| >= 32 (weights of
    several hundred), next to ordinary ones: the integer fragments q * sc and
    the fp32 factors do not depend on the magnitude, so every row group
    matches the fp64 reference on its own scale on every route."""
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(44)
    N, K, M = 96, 1024, 4
    w = rng.normal(0, 0.02, size=(N, K)).astype(np.float32)
    w[5, 256:512] *= 3e4      # one super-block of row 5 (|w| up to about 2e3)
    w[40:48, :256] *= 1e4     # the first super-block of rows 40..47
    wire = okq.quantize(w, "q4_k")
    x = fp16_rows(rng, M, K)
    ref = okq.qmm_ref(x, wire, "q4_k")
    for name, env in WIDE_ROUTES:
        for k in PATH_KNOBS + ("GMLX_KQ_MM", "GMLX_KQ_MMS"):
            monkeypatch.delenv(k, raising=False)
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        got = ops.quantized_matmul(_dev(x), _dev(wire), None, "q4_k", out_dtype=torch.float32).cpu().numpy()
        for rows in ([5], list(range(40, 48)), [n for n in range(N) if n != 5 and not 40 <= n < 48]):
            assert okq.max_rel(got[:, rows], ref[:, rows]) <= TOL, (name, rows)


WIDE_ROUTES = [("default", {}), ("stream", {"GMLX_KQ_STREAM": "2"}),
               ("mv", {"GMLX_KQ_STREAM": "0", "GMLX_KQ_MV": "2"}),
               ("dense", {"GMLX_KQ_STREAM": "0", "GMLX_KQ_MV": "0", "GMLX_KQ_MM": "0", "GMLX_KQ_MMS": "0"}),
               ("mid-batch tile", {"GMLX_KQ_MMS": "0"}),
               ("mid-batch streaming", {"GMLX_KQ_MMS": "2"})]


@pytest.mark.parametrize("M", [1, 7, 24, 80])
@pytest.mark.parametrize("codec", ["q4_k", "q6_k", "iq2_xxs"])
def test_wide_range_activations(M, codec, monkeypatch):
    """bf16 and fp32 activation rows far outside fp16's range -- entries of a
    few 1e5, rows scaled by 1e-6 (below fp16's 2^-14 normal limit) -- through
    every route (M 1 / 7: streaming, LDS-staged; 24: the mid-batch tile
    kernel and, forced, the mid-batch streaming kernel in K slices; 80 and
    the forced route: general).  Each row enters as fp16
    with a power of two of its own and its results are scaled back in fp32,
    so every output row matches the fp64 reference on its own scale
    (narrowing straight to fp16 turned the first row to inf and the second
    to zeros).  bf16 values are exact after the scaling; fp32 ones round once
    to 11 bits."""
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(M * 7 + len(codec))
    N, K = 160, 1024
    if codec == "iq2_xxs":
        wire = okq.random_valid_blocks(rng, codec, N * K // 256).reshape(N, -1)
    else:
        wire = quantized_weights(rng, codec, N, K)
    x = rng.normal(0.0, 1.0, size=(M, K)).astype(np.float32)
    x[0] *= 1e5
    if M > 1:
        x[1] *= 1e-6
        x[-1, 5] = 3.0e5
    for dt in (torch.bfloat16, torch.float32):
        xd = torch.from_numpy(x).to(dt)
        ref = okq.qmm_ref(xd.float().numpy(), wire, codec)
        for name, env in WIDE_ROUTES:
            if name in ("stream", "mv") and M > 16:
                continue
            for k in PATH_KNOBS + ("GMLX_KQ_MM", "GMLX_KQ_MMS"):
                monkeypatch.delenv(k, raising=False)
            for k, v in env.items():
                monkeypatch.setenv(k, v)
            got = ops.quantized_matmul(xd.cuda(), _dev(wire), None, codec, out_dtype=torch.float32).cpu().numpy()
            assert np.all(np.isfinite(got)), (name, dt)
            for m in range(M):
                err = okq.max_rel(got[m], ref[m])
                assert err <= TOL, (name, dt, m, err)


@pytest.mark.parametrize("codec", ["q4_k", "q6_k", "iq2_xxs"])
@pytest.mark.parametrize("M", [4, 24])
def test_large_fp16_activations_every_route(codec, M, monkeypatch):
    """fp16 activations of a few 1e4 (sums of 32 of them pass 65504): the
    Q4_K minimum term's activation sub-block sums are fp32; every route
    stays finite and within tolerance."""
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(91)
    N, K = 96, 2048
    if codec == "iq2_xxs":
        wire = okq.random_valid_blocks(rng, codec, N * K // 256).reshape(N, -1)
    else:
        wire = quantized_weights(rng, codec, N, K)
    x = np.clip(rng.normal(0.0, 1.0, size=(M, K)) * 15000.0, -60000, 60000).astype(np.float16)
    ref = okq.qmm_ref(x, wire, codec)
    for name, env in WIDE_ROUTES:
        if name in ("stream", "mv") and M > 16:
            continue
        for k in PATH_KNOBS + ("GMLX_KQ_MM", "GMLX_KQ_MMS"):
            monkeypatch.delenv(k, raising=False)
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        got = ops.quantized_matmul(_dev(x), _dev(wire), None, codec, out_dtype=torch.float32).cpu().numpy()
        assert np.all(np.isfinite(got)), name
        assert okq.max_rel(got, ref) <= TOL, (name, okq.max_rel(got, ref))


@pytest.mark.parametrize("codec", ["q4_k", "q6_k", "iq2_xxs"])
@pytest.mark.parametrize("M", [1, 8, 16, 24, 64])
def test_one_signed_rows_every_route(codec, M, monkeypatch):
    """Strongly one-signed fp16 activation rows (mean 2e4, std 1.2e4): every
    weight's error adds up coherently over such a row, so a weight that is
    not the reference's exact value (a scale or minimum rounded to fp16)
    shows here first.  The MFMA fragments are exact integers and the scales
    and minima fp32, so every route stays within the north-star max-rel by
    the reference's metric (max |err| / max |ref|, tests/test_ragged_decode.py:78-81)."""
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(1000 + M)
    N, K = 160, 4096
    if codec == "iq2_xxs":
        wire = okq.random_valid_blocks(rng, codec, N * K // 256).reshape(N, -1)
    else:
        wire = quantized_weights(rng, codec, N, K)
    x = np.clip(rng.normal(2e4, 1.2e4, size=(M, K)), -60000, 60000).astype(np.float16)
    ref = okq.qmm_ref(x, wire, codec)
    for name, env in WIDE_ROUTES:
        if name in ("stream", "mv") and M > 16:
            continue
        for k in PATH_KNOBS + ("GMLX_KQ_MM", "GMLX_KQ_MMS"):
            monkeypatch.delenv(k, raising=False)
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        got = ops.quantized_matmul(_dev(x), _dev(wire), None, codec, out_dtype=torch.float32).cpu().numpy()
        assert okq.max_rel(got, ref) <= TOL, (name, okq.max_rel(got, ref))
