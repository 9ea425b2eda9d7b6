"""Host drivers of the batched-decode attention path.

Which rows are live, how many decode together, which kernel claims an
attention call, and the shared-prefix stamp that makes a batch eligible for
the cascade kernel.  Everything here is host logic on Python objects and
int lists; the only device work is the op call a claim makes.

Reference behaviour mirrored:
  batch_rows / batch_rows_of        gmlx/batch_rows.py:20-39
  decode_batch                      gmlx/decode_batch.py:27-39
  cascade claim gates and slicing   gmlx/cascade_sdpa.py:79-124, 136-260
  route wrapper / seam install      gmlx/cascade_sdpa.py:263-305
  stamp lifecycle                   gmlx/cascade_sdpa.py:324-543
  left-padded route order           gmlx/qwen35_attn.py:583-616

Caches are duck-typed like the reference's batch KV caches: `left_padding`
(a tensor or int sequence), optional `extend(other)` / `filter(keep)`, an
optional `bits` attribute marking a quantised cache.  The stamp lives in the
cache's `_gmlx_cascade` attribute as {"P": shared token count, "tok": per-row
packed token bytes}, the reference's own attribute and format, so a cache
stamped by either side reads the same.

Claims only ever decline: any rejection (shape, dtype, a kernel error)
returns None and the caller runs its stock attention.  Nothing here reads a
device value on the host except the pads, once per `left_padding` object.
"""
from __future__ import annotations

import array
import os
import sys

DEFAULT_DECODE_BATCH = 8
UPSTREAM_DECODE_BATCH = 32      # the serving engine's own hard-wired default
CASCADE_HEAD_DIMS = (64, 128, 256)  # the reference's (64, 128, 256, 512) minus 512, which the kernel lacks

_CLAIMS = [0]
_STAMPS = [0]
_DEBUG_LINES = [0]


# --------------------------------------------------------------- env flags

def _env_bool(name, default):
    raw = os.environ.get(name, "").strip().lower()
    if not raw:
        return default
    return raw not in ("0", "false", "no", "off")


def _env_int(name, default):
    raw = os.environ.get(name, "").strip()
    try:
        return int(raw) if raw else default
    except ValueError:
        return default


# --------------------------------------------------------------- live rows

def batch_rows_of(batch) -> int:
    """Active rows of a generation batch without side effects.  A batch with
    `_finished` flags (the speculative batch, whose __len__ may promote a
    buffered injection) is counted from the flags; others by len()."""
    if batch is None:
        return 0
    flags = getattr(batch, "_finished", None)
    if flags is not None:
        return sum(not done for done in flags)
    return len(batch)


def batch_rows(gen) -> int:
    """Active rows of `gen._generation_batch`; 0 when there is none."""
    return batch_rows_of(getattr(gen, "_generation_batch", None))


def decode_batch() -> int:
    """Decode concurrency (GMLX_DECODE_BATCH): a positive value is used as
    given, 0 selects the engine's own default, anything else (unset, not a
    number, negative) the default of 8."""
    raw = os.environ.get("GMLX_DECODE_BATCH", "").strip()
    if not raw:
        return DEFAULT_DECODE_BATCH
    try:
        n = int(raw)
    except ValueError:
        return DEFAULT_DECODE_BATCH
    if n > 0:
        return n
    return UPSTREAM_DECODE_BATCH if n == 0 else DEFAULT_DECODE_BATCH


# ------------------------------------------------------------- counters

def claims() -> int:
    """Attention calls the cascade route has claimed since import."""
    return _CLAIMS[0]


def stamps() -> int:
    """Batches stamped with a shared prefix since import."""
    return _STAMPS[0]


def _decline(reason, **kw):
    """GMLX_CASCADE_DEBUG=1 prints the first GMLX_CASCADE_DEBUG_N declines."""
    if os.environ.get("GMLX_CASCADE_DEBUG") == "1" and _DEBUG_LINES[0] < _env_int("GMLX_CASCADE_DEBUG_N", 8):
        _DEBUG_LINES[0] += 1
        print(f"[cascade] decline: {reason} {kw}", file=sys.stderr, flush=True)
    return None


# ------------------------------------------------------- pads and starts

def _host_ints(x):
    if hasattr(x, "tolist"):
        return [int(v) for v in x.tolist()]
    return [int(v) for v in x]


def cache_pads(cache):
    """Per-row left padding as host ints, read once per `left_padding`
    object (batch changes rebind the attribute, so identity is the key)."""
    lp = getattr(cache, "left_padding", None)
    if lp is None:
        return None
    memo = cache.__dict__.get("_gmlx_casc_pads")
    if memo is not None and memo[0] is lp:
        return memo[1]
    pads = _host_ints(lp)
    cache._gmlx_casc_pads = (lp, pads)
    return pads


def cascade_starts(cache, pads, P, device):
    """(starts, c0) for a stamped cache: the private slab begins at
    c0 = min(pads) + P and row b's private keys at starts[b] = pads[b] + P - c0
    inside it.  `starts` is an int32 device tensor, memoised with the pads."""
    import torch
    lp = cache.left_padding
    memo = cache.__dict__.get("_gmlx_casc_starts")
    if memo is not None and memo[0] is lp and memo[1] == P and memo[2].device == device:
        return memo[2], memo[3]
    c0 = min(pads) + P
    starts = torch.tensor([p + P - c0 for p in pads], dtype=torch.int32, device=device)
    cache._gmlx_casc_starts = (lp, P, starts, c0)
    return starts, c0


def mask_claimable(mask, qL) -> bool:
    """Masks the cascade op reproduces: at decode width None, "causal" or a
    mask of width 1; at verify width "causal" or a mask of width qL (left
    padding plus the end-aligned causal of the block).  None at qL > 1 is an
    unmasked block, which the op does not compute."""
    if isinstance(mask, str):
        return mask == "causal"
    if mask is None:
        return qL == 1
    shape = getattr(mask, "shape", None)
    return shape is not None and len(shape) >= 2 and shape[-2] == qL


# ----------------------------------------------------------- the claim

def cascade_claim(queries, keys, values, cache, scale, mask=None, sinks=None):
    """Cascade output for a claimable stamped batched call, else None.

    queries (B, Hq, qL, D); keys/values the cache's (B, Hkv, L, D) buffers,
    each row holding the shared prefix at [pads[b], pads[b] + P).  The op
    runs on views of those buffers: the prefix is row 0's copy, the private
    slab starts at c0."""
    import torch
    info = cache.__dict__.get("_gmlx_cascade") if cache is not None and hasattr(cache, "__dict__") else None
    if info is None:
        return _decline("no-stamp")
    # 8-bit affine caches (bits 8, group 64) present K / V as (wire, scales,
    # biases); other quantized configurations decline
    quant = (isinstance(keys, (tuple, list)) and len(keys) == 3 and isinstance(values, (tuple, list))
             and len(values) == 3 and getattr(cache, "bits", None) == 8
             and getattr(cache, "group_size", None) == 64)
    if not quant and (isinstance(keys, (tuple, list)) or getattr(cache, "bits", None) is not None):
        return _decline("quant-config", bits=getattr(cache, "bits", None), gs=getattr(cache, "group_size", None))
    ka = keys[0] if quant else keys
    va = values[0] if quant else values
    if not all(isinstance(t, torch.Tensor) for t in (queries, ka, va)):
        return _decline("not-tensors")
    if queries.dim() != 4 or ka.dim() != 4 or va.dim() != 4:
        return _decline("rank")
    B, Hq, qL, D = queries.shape
    Hkv, kL = ka.shape[1], ka.shape[2]
    kv_last = D // 4 if quant else D
    dt_ok = ((ka.dtype in (torch.int32, getattr(torch, "uint32", torch.int32)) and keys[1].dtype == queries.dtype)
             if quant else (ka.dtype == queries.dtype and va.dtype == queries.dtype))
    if not (sinks is None and B > 1 and 1 <= qL <= 8 and D in CASCADE_HEAD_DIMS
            and ka.shape[0] == B and tuple(va.shape) == tuple(ka.shape) and ka.shape[3] == kv_last
            and Hkv >= 1 and Hq % Hkv == 0
            and queries.dtype in (torch.float16, torch.bfloat16) and dt_ok
            and getattr(cache, "_right_padding", None) is None and mask_claimable(mask, qL)):
        return _decline("shape/dtype/mask", B=B, qL=qL, D=D, dtype=str(queries.dtype), quant=quant)
    G = Hq // Hkv
    if G > 16 or B * G * qL > 64:
        return _decline("width", G=G, B=B, qL=qL)
    if qL > 1 and G * ((qL + 1) // 2) > 32:
        return _decline("verify-width", G=G, qL=qL)
    P = int(info["P"])
    if P < _env_int("GMLX_CASCADE_MIN_P", 1024):
        return _decline("short-prefix", P=P)
    pads = cache_pads(cache)
    if pads is None or len(pads) < B:
        return _decline("pads")
    pads = pads[:B]
    c0 = min(pads) + P
    if kL - c0 < qL or max(pads) + P > kL - qL + 1:
        return _decline("geometry", kL=kL, c0=c0, P=P)
    from . import ops
    from ._lib import KQLibraryError
    try:
        starts, c0 = cascade_starts(cache, pads, P, queries.device)
        l0 = pads[0]
        sh = lambda t: t[0:1, :, l0:l0 + P]  # noqa: E731  row 0's prefix copy
        pr = lambda t: t[:, :, c0:]  # noqa: E731  the private slab
        if quant:
            kw, ks, kb = keys
            vw, vs, vb = values
            out = ops.sdpa_decode_gqa_cascade(
                queries, sh(kw), sh(vw), pr(kw), pr(vw), scale, starts=starts,
                k_shared_scales=sh(ks), k_shared_biases=sh(kb), v_shared_scales=sh(vs), v_shared_biases=sh(vb),
                k_priv_scales=pr(ks), k_priv_biases=pr(kb), v_priv_scales=pr(vs), v_priv_biases=pr(vb))
        else:
            out = ops.sdpa_decode_gqa_cascade(queries, sh(keys), sh(values), pr(keys), pr(values), scale,
                                              starts=starts)
    except KQLibraryError:
        raise  # a missing library is a broken install, not a declined call
    except Exception as e:  # the route only declines
        return _decline("kernel", err=str(e)[:120])
    _CLAIMS[0] += 1
    return out


def make_route(orig):
    """Wrap a module-global attention seam `orig(queries, keys, values,
    cache=None, scale=1.0, mask=None, sinks=None)`: claimed calls run the
    cascade op, everything else goes to `orig` unchanged."""
    def cascade_sdpa(queries, keys, values, cache=None, scale=1.0, mask=None, sinks=None):
        out = cascade_claim(queries, keys, values, cache, scale, mask, sinks)
        if out is not None:
            return out
        return orig(queries, keys, values, cache=cache, scale=scale, mask=mask, sinks=sinks)

    cascade_sdpa._gmlx_orig = orig
    cascade_sdpa._gmlx_cascade_route = True
    return cascade_sdpa


def install_cascade_sdpa(modules) -> bool:
    """Route the `scaled_dot_product_attention` seam of each given module
    through the cascade claim.  Idempotent; GMLX_CASCADE_SDPA=0 disables it.
    True when at least one seam is routed."""
    if not _env_bool("GMLX_CASCADE_SDPA", True):
        return False
    routed = 0
    for mod in modules:
        cur = getattr(mod, "scaled_dot_product_attention", None)
        if cur is None:
            continue
        if not getattr(cur, "_gmlx_cascade_route", False):
            mod.scaled_dot_product_attention = make_route(cur)
        routed += 1
    return routed > 0


def left_padded_attention(queries, keys, values, *, cache, scale, mask=None):
    """Route order for a left-padded batched decode call: the cascade claim
    (B > 1, qL 1, GMLX_CASCADE_SDPA on), then the ragged kernel; None when
    neither takes it (the caller's stock attention runs).  A quantised cache,
    non-4-D tensors or a batch without padding decline at once."""
    from . import ops
    if getattr(cache, "bits", None) is not None or getattr(queries, "dim", lambda: 0)() != 4 \
            or getattr(keys, "dim", lambda: 0)() != 4:
        return None
    pads = cache.__dict__.get("_qwen3_5_decode_left_padding") if hasattr(cache, "__dict__") else None
    if pads is None:
        pads = cache_pads(cache)
    if not pads or max(pads) <= 0:
        return None
    if queries.shape[0] > 1 and queries.shape[2] == 1 and _env_bool("GMLX_CASCADE_SDPA", True):
        out = cascade_claim(queries, keys, values, cache, scale, None, None)
        if out is not None:
            return out
    from ._lib import KQLibraryError
    try:
        return ops.ragged_decode_attention(queries, keys, values, list(pads), scale)
    except KQLibraryError:
        raise
    except Exception as e:
        return _decline("ragged", err=str(e)[:120])


# ------------------------------------------------------- prefix stamps

def row_bytes(ids) -> bytes:
    """A row's token ids packed as int32 bytes: rows compare by memcmp."""
    return array.array("i", [int(t) for t in ids]).tobytes()


def lcp_rows(rows) -> int:
    """Tokens in the longest prefix common to all packed rows (0 if any row
    is empty or there are none)."""
    if not rows or any(len(r) == 0 for r in rows):
        return 0
    return len(os.path.commonprefix(list(rows))) // 4


def merge_stamps(a, b):
    """Stamp of the batch extend() forms (a's rows, then b's): the common
    prefix of the two sides' shared prefixes, or None."""
    if a is None or b is None:
        return None
    P = lcp_rows([a["tok"][0][:4 * a["P"]], b["tok"][0][:4 * b["P"]]])
    return {"P": P, "tok": tuple(a["tok"]) + tuple(b["tok"])} if P > 0 else None


def _keep_stamp_on_extend(cache):
    fn = getattr(cache, "extend", None)
    if fn is None or getattr(fn, "_gmlx_cascade_merge", False):
        return

    def extend(other, _cache=cache, _orig=fn):
        merged = merge_stamps(_cache.__dict__.get("_gmlx_cascade"), getattr(other, "_gmlx_cascade", None))
        out = _orig(other)
        if merged is None:
            _cache.__dict__.pop("_gmlx_cascade", None)
        else:
            _cache._gmlx_cascade = merged
        return out

    extend._gmlx_cascade_merge = True
    cache.extend = extend


def _keep_stamp_on_filter(cache):
    fn = getattr(cache, "filter", None)
    if fn is None or getattr(fn, "_gmlx_cascade_filter", False):
        return

    def filter_rows(keep, *args, _cache=cache, _orig=fn, **kw):
        info = _cache.__dict__.get("_gmlx_cascade")
        out = _orig(keep, *args, **kw)
        if info is not None:
            kept = tuple(t for t, k in zip(info["tok"], _host_ints(keep) if hasattr(keep, "tolist") else keep) if k)
            if kept:
                _cache._gmlx_cascade = {"P": info["P"], "tok": kept}
            else:
                _cache.__dict__.pop("_gmlx_cascade", None)
        return out

    filter_rows._gmlx_cascade_filter = True
    cache.filter = filter_rows


def stamp_caches(caches, rows) -> bool:
    """Stamp every layer cache with the rows' shared token prefix (rows:
    packed token bytes in cache row order).  Returns False, stamping
    nothing, when the rows share no prefix."""
    P = lcp_rows(rows)
    if P <= 0:
        return False
    tok = tuple(rows)
    for c in caches:
        c._gmlx_cascade = {"P": P, "tok": tok}
        _keep_stamp_on_extend(c)
        _keep_stamp_on_filter(c)
    _STAMPS[0] += 1
    return True


def carry_stamp(src, dst):
    """Move a live stamp to a rebuilt cache object of the same rows."""
    st = src.__dict__.get("_gmlx_cascade") if src is not None else None
    if st is None or dst is None:
        return
    dst._gmlx_cascade = st
    _keep_stamp_on_extend(dst)
    _keep_stamp_on_filter(dst)


def rows_from_prompt_batch(pb):
    """Per-row full prompt tokens (packed) of a just-built prompt batch:
    from `_apc_meta[i]["full_input_ids"]` when the batch carries that meta
    (every row must have ids, else None), otherwise from the untouched
    `_input_ids` rows with each row's left / right padding stripped."""
    meta = getattr(pb, "_apc_meta", None)
    if meta:
        rows = []
        for m in meta:
            ids = (m or {}).get("full_input_ids")
            if not ids:
                return None
            rows.append(row_bytes(ids))
        return rows
    ids = getattr(pb, "_input_ids", None)
    lpad = getattr(pb, "_left_padding_per_row", None)
    if ids is None or lpad is None or len(getattr(ids, "shape", ())) != 2:
        return None
    rpad = getattr(pb, "_right_pad_per_row", None) or [0] * len(lpad)
    L = ids.shape[1]
    out = []
    for i, lp in enumerate(lpad):
        rp = rpad[i] if i < len(rpad) else 0
        out.append(row_bytes(_host_ints(ids[i, lp:L - rp])))
    return out


def _stamped_init(orig):
    def init(self, *args, **kw):
        orig(self, *args, **kw)
        try:
            caches = getattr(self, "prompt_cache", None)
            rows = rows_from_prompt_batch(self) if caches else None
            if rows:
                stamp_caches(caches, rows)
            else:
                _decline("stamp-no-rows")
        except Exception as e:  # stamping never breaks batch formation
            _decline("stamp", err=str(e)[:120])

    init._gmlx_orig = orig
    init._gmlx_cascade_stamp = True
    return init


def _stamped_extend_cache(orig):
    def extend_cache(a, b):
        pairs = [(getattr(ca, "_gmlx_cascade", None), getattr(cb, "_gmlx_cascade", None)) for ca, cb in zip(a, b)]
        out = orig(a, b)
        for oc, (sa, sb) in zip(out, pairs):
            merged = merge_stamps(sa, sb)
            if merged is None:
                oc.__dict__.pop("_gmlx_cascade", None)
            else:
                oc._gmlx_cascade = merged
                _keep_stamp_on_extend(oc)
                _keep_stamp_on_filter(oc)
        return out

    extend_cache._gmlx_orig = orig
    extend_cache._gmlx_cascade_stamp = True
    return extend_cache


def install_cascade_stamp(engine_module) -> bool:
    """Stamp batches at formation in a serving engine module exposing
    `PromptProcessingBatch` and `_extend_cache` (the reference patches its
    engine's module of those names).  Idempotent; GMLX_CASCADE_SDPA=0
    disables it."""
    if not _env_bool("GMLX_CASCADE_SDPA", True):
        return False
    ppb = getattr(engine_module, "PromptProcessingBatch", None)
    ext = getattr(engine_module, "_extend_cache", None)
    if ppb is None or ext is None:
        return False
    if not getattr(ppb.__init__, "_gmlx_cascade_stamp", False):
        ppb.__init__ = _stamped_init(ppb.__init__)
    if not getattr(ext, "_gmlx_cascade_stamp", False):
        engine_module._extend_cache = _stamped_extend_cache(ext)
    return True
