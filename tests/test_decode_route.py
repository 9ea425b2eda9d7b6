"""Host drivers of the decode path (gmlx_amd.decode_route): live-row counts,
decode concurrency, cascade claim gates and the shared-prefix stamp
lifecycle.  Pure host logic, mirroring the reference's always-run tests
(tests/test_cascade_sdpa.py stamp tests, tests/test_batch_rows.py,
tests/test_decode_batch.py); kernel numerics of claimed calls are in
test_gpu_cascade.py."""
import types

import pytest
import torch

from gmlx_amd import decode_route as dr


class _Cache:
    """Batch-cache stand-in: left padding, optional stamp, extend/filter."""

    def __init__(self, pads, P=None):
        self.left_padding = torch.tensor(pads)
        self._right_padding = None
        if P is not None:
            self._gmlx_cascade = {"P": P, "tok": ()}

    def extend(self, other):
        return "extended"

    def filter(self, keep):
        return "filtered"


def _rb(ids):
    return dr.row_bytes(ids)


# ------------------------------------------------------------- rows / batch

def test_batch_rows_counts_unfinished_without_len():
    class Spec:
        _finished = [False, True, False, False]

        def __len__(self):
            raise AssertionError("len() promotes on a spec batch")

    assert dr.batch_rows_of(Spec()) == 3
    assert dr.batch_rows_of([1, 2]) == 2
    assert dr.batch_rows_of(None) == 0
    assert dr.batch_rows(types.SimpleNamespace(_generation_batch=Spec())) == 3
    assert dr.batch_rows(object()) == 0


@pytest.mark.parametrize("raw,want", [("", 8), ("4", 4), ("0", 32), ("-3", 8), ("x", 8), (" 16 ", 16)])
def test_decode_batch_env(monkeypatch, raw, want):
    monkeypatch.setenv("GMLX_DECODE_BATCH", raw)
    assert dr.decode_batch() == want


# ------------------------------------------------------------------ stamps

def test_lcp_rows():
    a = list(range(100))
    assert dr.lcp_rows([_rb(a), _rb(a)]) == 100
    assert dr.lcp_rows([_rb(a), _rb(a[:50] + [999] + a[51:])]) == 50
    assert dr.lcp_rows([_rb(a), _rb(a[:30])]) == 30
    assert dr.lcp_rows([_rb(a)]) == 100
    assert dr.lcp_rows([]) == 0
    assert dr.lcp_rows([_rb(a), b""]) == 0
    # a common byte prefix inside a token does not count as a token
    assert dr.lcp_rows([_rb([1, 2, 0x100]), _rb([1, 2, 0x200])]) == 2


def test_stamp_caches_and_merge_on_extend():
    pre = list(range(64))
    cache = _Cache([0, 0])
    n0 = dr.stamps()
    assert dr.stamp_caches([cache], [_rb(pre + [1]), _rb(pre + [2])])
    assert dr.stamps() == n0 + 1
    assert cache._gmlx_cascade["P"] == 64
    other = _Cache([0])
    dr.stamp_caches([other], [_rb(pre[:40] + [999])])
    assert cache.extend(other) == "extended"
    assert cache._gmlx_cascade["P"] == 40
    assert len(cache._gmlx_cascade["tok"]) == 3
    # an unstamped side clears the stamp
    assert cache.extend(_Cache([0])) == "extended"
    assert not hasattr(cache, "_gmlx_cascade")


def test_stamp_divergent_clears():
    cache = _Cache([0])
    dr.stamp_caches([cache], [_rb([1, 2, 3])])
    other = _Cache([0])
    dr.stamp_caches([other], [_rb([9, 9, 9])])
    cache.extend(other)
    assert not hasattr(cache, "_gmlx_cascade")


def test_stamp_no_common_prefix_no_stamp():
    cache = _Cache([0, 0])
    assert not dr.stamp_caches([cache], [_rb([1, 2]), _rb([3, 4])])
    assert not hasattr(cache, "_gmlx_cascade")


def test_stamp_filter_masks_rows():
    cache = _Cache([0, 0, 0])
    rows = [_rb(list(range(32)) + [i]) for i in range(3)]
    dr.stamp_caches([cache], rows)
    assert cache.filter([True, False, True]) == "filtered"
    info = cache._gmlx_cascade
    assert info["P"] == 32 and info["tok"] == (rows[0], rows[2])
    assert cache.filter(torch.tensor([False, False])) == "filtered"
    assert not hasattr(cache, "_gmlx_cascade")


def test_wrappers_install_once():
    cache = _Cache([0, 0])
    dr.stamp_caches([cache], [_rb([1, 2]), _rb([1, 3])])
    ext, flt = cache.extend, cache.filter
    dr.stamp_caches([cache], [_rb([1, 2]), _rb([1, 3])])
    assert cache.extend is ext and cache.filter is flt


def test_carry_stamp():
    src = _Cache([0, 0])
    dr.stamp_caches([src], [_rb([5, 6, 7]), _rb([5, 6, 8])])
    dst = _Cache([0, 0])
    dr.carry_stamp(src, dst)
    assert dst._gmlx_cascade == src._gmlx_cascade
    assert getattr(dst.extend, dr.HOOK_MARK, False)
    dst2 = _Cache([0, 0])
    dr.carry_stamp(_Cache([0, 0]), dst2)
    assert "_gmlx_cascade" not in dst2.__dict__


def test_rows_from_prompt_batch_cold_and_meta():
    ids = torch.tensor([[0, 0, 7, 8, 9], [7, 8, 9, 10, 0]])
    pb = types.SimpleNamespace(_apc_meta=[], _input_ids=ids, _left_padding_per_row=[2, 0],
                               _right_pad_per_row=[0, 1])
    assert dr.rows_from_prompt_batch(pb) == [_rb([7, 8, 9]), _rb([7, 8, 9, 10])]
    pb = types.SimpleNamespace(_apc_meta=[{"full_input_ids": [1, 2]}, {"full_input_ids": [1, 3]}])
    assert dr.rows_from_prompt_batch(pb) == [_rb([1, 2]), _rb([1, 3])]
    pb = types.SimpleNamespace(_apc_meta=[{"full_input_ids": [1, 2]}, {}])
    assert dr.rows_from_prompt_batch(pb) is None
    assert dr.rows_from_prompt_batch(types.SimpleNamespace()) is None


def test_install_cascade_stamp_on_an_engine_module(monkeypatch):
    class PPB:
        def __init__(self, caches, ids, pads):
            self.prompt_cache = caches
            self._apc_meta = None
            self._input_ids = ids
            self._left_padding_per_row = pads

    def _extend_cache(a, b):
        return [_Cache([0, 0, 0]) for _ in a]

    eng = types.SimpleNamespace(PromptProcessingBatch=PPB, _extend_cache=_extend_cache)
    assert dr.install_cascade_stamp(eng)
    assert dr.install_cascade_stamp(eng)          # idempotent
    caches = [_Cache([1, 0]), _Cache([1, 0])]
    PPB(caches, torch.tensor([[0, 4, 5, 6], [4, 5, 6, 7]]), [1, 0])
    assert all(c._gmlx_cascade["P"] == 3 for c in caches)
    one = [_Cache([0])]
    dr.stamp_caches(one, [_rb([4, 5, 9])])
    merged = eng._extend_cache(caches[:1], one)
    assert merged[0]._gmlx_cascade["P"] == 2 and len(merged[0]._gmlx_cascade["tok"]) == 3
    monkeypatch.setenv("GMLX_CASCADE_SDPA", "0")
    assert not dr.install_cascade_stamp(types.SimpleNamespace(PromptProcessingBatch=PPB, _extend_cache=_extend_cache))


# ------------------------------------------------------------------- claim

def test_mask_claimable():
    assert dr.mask_claimable(None, 1) and not dr.mask_claimable(None, 4)
    assert dr.mask_claimable("causal", 4) and not dr.mask_claimable("full", 1)
    assert dr.mask_claimable(torch.zeros(2, 1, 4, 100, dtype=torch.bool), 4)
    assert not dr.mask_claimable(torch.zeros(2, 1, 1, 100, dtype=torch.bool), 4)


def test_pads_and_starts_memoised_on_pad_identity():
    cache = _Cache([0, 64, 128, 32], P=1024)
    pads = dr.cache_pads(cache)
    assert pads == [0, 64, 128, 32] and dr.cache_pads(cache) is pads
    starts, c0 = dr.cascade_starts(cache, pads, 1024, torch.device("cpu"))
    assert c0 == 1024 and starts.tolist() == [0, 64, 128, 32] and starts.dtype == torch.int32
    again, _ = dr.cascade_starts(cache, pads, 1024, torch.device("cpu"))
    assert again is starts                              # the device table is built once
    cache.left_padding = torch.tensor([3, 1, 2, 9])     # a new pads object: recomputed
    pads = dr.cache_pads(cache)
    fresh, c0 = dr.cascade_starts(cache, pads, 1024, torch.device("cpu"))
    assert fresh is not starts and c0 == 1025 and fresh.tolist() == [2, 0, 1, 8]


def _qkv(B=4, Hq=16, Hkv=8, qL=1, L=1200, D=128, dtype=torch.float16):
    return (torch.zeros(B, Hq, qL, D, dtype=dtype), torch.zeros(B, Hkv, L, D, dtype=dtype),
            torch.zeros(B, Hkv, L, D, dtype=dtype))


@pytest.mark.parametrize("case", ["no-stamp", "B1", "qL9", "D96", "fp32", "short-prefix", "geometry",
                                  "quant", "mask-None-verify", "sinks", "gqa17", "wide", "wide512", "right-pad"])
def test_claim_declines(monkeypatch, case):
    q, k, v = _qkv()
    cache = _Cache([0, 4, 8, 2], P=1024)
    kw = {}
    if case == "no-stamp":
        cache = _Cache([0, 4, 8, 2])
    elif case == "B1":
        q, k, v = _qkv(B=1)
        cache = _Cache([0], P=1024)
    elif case == "qL9":
        q, k, v = _qkv(qL=9)
        kw["mask"] = "causal"
    elif case == "D96":
        q, k, v = _qkv(D=96)
    elif case == "fp32":
        q, k, v = _qkv(dtype=torch.float32)
    elif case == "short-prefix":
        monkeypatch.setenv("GMLX_CASCADE_MIN_P", "2048")
    elif case == "geometry":
        cache = _Cache([0, 4, 180, 2], P=1024)           # max(pads) + P > L - qL + 1
    elif case == "quant":
        cache.bits = 4                                    # only 8-bit group-64 caches are claimed
        cache.group_size = 64
        k = (k, torch.zeros(4, 8, 1200, 2, dtype=torch.float16), torch.zeros(4, 8, 1200, 2, dtype=torch.float16))
        v = k
    elif case == "mask-None-verify":
        q, k, v = _qkv(qL=4)
    elif case == "sinks":
        kw["sinks"] = torch.zeros(16)
    elif case == "gqa17":
        q, k, v = _qkv(Hq=17 * 8)
    elif case == "wide":
        q, k, v = _qkv(B=8, Hq=32, qL=4)                 # B * G * qL = 128 > 64
        kw["mask"] = "causal"
    elif case == "wide512":
        q, k, v = _qkv(B=8, Hq=16, Hkv=8, qL=4, D=512)   # B * G * qL = 64 > 32 at head dim 512
        kw["mask"] = "causal"
    elif case == "right-pad":
        cache._right_padding = [0, 1, 0, 0]
    n0 = dr.claims()
    assert dr.cascade_claim(q, k, v, cache, 0.088, kw.get("mask"), kw.get("sinks")) is None
    assert dr.claims() == n0


@pytest.mark.parametrize("D,want", [(512, "quant-config"), (128, "kernel")])
def test_q8_cache_declines_at_head_dim_512(monkeypatch, capsys, D, want):
    """An 8-bit group-64 cache is claimed at head dims other than 512 and
    declines at 512 as the reference's gate does (gmlx/cascade_sdpa.py:150-157,
    'and hd != 512'): the 512 call stops at the quantisation gate, the 128
    call passes every gate and reaches the op (which rejects CPU tensors)."""
    monkeypatch.setenv("GMLX_CASCADE_DEBUG", "1")
    monkeypatch.setenv("GMLX_CASCADE_DEBUG_N", "1000000")
    B, Hq, Hkv, qL, L = 4, 16, 8, 1, 1200
    q = torch.zeros(B, Hq, qL, D, dtype=torch.float16)
    words = torch.zeros(B, Hkv, L, D // 4, dtype=torch.int32)
    sc = torch.zeros(B, Hkv, L, D // 64, dtype=torch.float16)
    cache = _Cache([0, 4, 8, 2], P=1024)
    cache.bits = 8
    cache.group_size = 64
    n0 = dr.claims()
    assert dr.cascade_claim(q, (words, sc, sc), (words, sc, sc), cache, 0.088, None, None) is None
    assert dr.claims() == n0
    assert f"declined ({want})" in capsys.readouterr().err


def test_route_falls_through_to_orig_on_decline():
    calls = []

    def stock(queries, keys, values, cache=None, scale=1.0, mask=None, sinks=None):
        calls.append((cache, scale, mask))
        return "stock"

    mod = types.SimpleNamespace(scaled_dot_product_attention=stock)
    assert dr.install_cascade_sdpa([mod, types.SimpleNamespace()])
    route = mod.scaled_dot_product_attention
    assert route.orig is stock
    assert dr.install_cascade_sdpa([mod]) and mod.scaled_dot_product_attention is route   # idempotent
    q, k, v = _qkv()
    n0 = dr.claims()
    # stamped and claimable on the host, but CPU tensors: the op rejects, the route declines
    assert route(q, k, v, cache=_Cache([0, 4, 8, 2], P=1024), scale=0.5, mask=None) == "stock"
    assert route(q, k, v, cache=None, scale=0.5) == "stock"
    assert dr.claims() == n0 and len(calls) == 2


def test_install_killed_by_env(monkeypatch):
    monkeypatch.setenv("GMLX_CASCADE_SDPA", "0")
    mod = types.SimpleNamespace(scaled_dot_product_attention=lambda *a, **k: None)
    assert not dr.install_cascade_sdpa([mod])
    assert not isinstance(mod.scaled_dot_product_attention, dr._CascadeRoute)


def test_left_padded_route_declines_without_padding_or_for_quant():
    q, k, v = _qkv()
    assert dr.left_padded_attention(q, k, v, cache=_Cache([0, 0, 0, 0], P=1024), scale=0.1) is None
    qc = _Cache([0, 4, 8, 2], P=1024)
    qc.bits = 8
    assert dr.left_padded_attention(q, k, v, cache=qc, scale=0.1) is None
