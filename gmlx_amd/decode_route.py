"""Host side of the batched-decode attention path.

Four concerns, each a small object or function family:

* live rows and decode concurrency -- how many rows a batch holds and how
  many decode together (`batch_rows`, `batch_rows_of`, `decode_batch`);
* the shared-prefix stamp -- a `PrefixStamp` value (the token prefix every
  row of a batch shares, and the rows' packed tokens) kept on each layer
  cache and carried through the cache's `extend` / `filter`;
* the row geometry of a left-padded cache -- per-row pads read once per
  `left_padding` object, and the device table of private-slab starts;
* the claim -- an ordered list of gates a stamped attention call must pass
  before the cascade kernel takes it; every failure declines (returns None)
  and the caller runs its stock attention.

What must stay as the reference has it, so that either side reads the
other's work (interop, not structure):
  the stamp attribute `_gmlx_cascade` holding {"P": shared tokens, "tok":
  tuple of per-row int32 token bytes}          gmlx/cascade_sdpa.py:324-360
  the claim gates (head dims 64/128/256/512, GQA <= 16, B*G*qL <= 64, or
  32 at head dim 512, G*ceil(qL/2) <= 32 when verifying, qL <= 8, prefix
  >= GMLX_CASCADE_MIN_P tokens, 8-bit group-64 quantised caches only)
                                               gmlx/cascade_sdpa.py:136-224
  the slab formulas c0 = min(pads) + P, starts[b] = pads[b] + P - c0
                                               gmlx/cascade_sdpa.py:95-105
  the environment knobs GMLX_CASCADE_SDPA, GMLX_CASCADE_MIN_P,
  GMLX_CASCADE_DEBUG(_N), GMLX_DECODE_BATCH    gmlx/cascade_sdpa.py,
                                               gmlx/decode_batch.py:27-39
  live-row counting (`_finished` flags before len())
                                               gmlx/batch_rows.py:20-39

Caches are duck-typed like the reference's batch KV caches: `left_padding`
(a tensor or int sequence), optional `extend(other)` / `filter(keep)`, an
optional `bits` / `group_size` marking a quantised cache.  Nothing here reads
a device value on the host except the pads, once per `left_padding` object.
"""
from __future__ import annotations

import os
import sys
from dataclasses import dataclass
from typing import Optional, Sequence, Tuple

import numpy as np

STAMP_ATTR = "_gmlx_cascade"            # interop: the reference's attribute name and format
HOOK_MARK = "_kq_stamp_hooked"          # this module's private marker on hooked cache methods
GEOMETRY_ATTR = "_kq_row_geometry"      # this module's private per-cache memo

DEFAULT_DECODE_BATCH = 8
UPSTREAM_DECODE_BATCH = 32              # the serving engine's own hard-wired default
CASCADE_HEAD_DIMS = (64, 128, 256, 512)


class _Counters:
    claims = 0
    stamps = 0
    debug_lines = 0


# ------------------------------------------------------------------- knobs

def _flag(name: str, default: bool) -> bool:
    raw = os.environ.get(name, "").strip().lower()
    return default if not raw else raw not in ("0", "false", "no", "off")


def _number(name: str, default: int) -> int:
    raw = os.environ.get(name, "").strip()
    if not raw:
        return default
    try:
        return int(raw)
    except ValueError:
        return default


def cascade_enabled() -> bool:
    """GMLX_CASCADE_SDPA (default on) turns the cascade route and stamping on."""
    return _flag("GMLX_CASCADE_SDPA", True)


def _decline(reason: str, **details):
    """Return None; with GMLX_CASCADE_DEBUG=1, report the first
    GMLX_CASCADE_DEBUG_N declines (default 8) on stderr."""
    if os.environ.get("GMLX_CASCADE_DEBUG") == "1" and _Counters.debug_lines < _number("GMLX_CASCADE_DEBUG_N", 8):
        _Counters.debug_lines += 1
        extra = ", ".join(f"{k}={v}" for k, v in details.items())
        print(f"gmlx_amd cascade declined ({reason}){': ' + extra if extra else ''}", file=sys.stderr, flush=True)
    return None


def claims() -> int:
    """Attention calls the cascade route has taken since import."""
    return _Counters.claims


def stamps() -> int:
    """Batches stamped with a shared prefix since import."""
    return _Counters.stamps


# ------------------------------------------------------ rows / concurrency

def batch_rows_of(batch) -> int:
    """Rows still decoding in `batch`.  A batch that tracks `_finished` flags
    (the speculative batch, whose len() may promote a buffered injection) is
    counted from the flags without calling len()."""
    if batch is None:
        return 0
    done = getattr(batch, "_finished", None)
    return len(batch) if done is None else len(done) - sum(bool(d) for d in done)


def batch_rows(gen) -> int:
    """Rows of a generator's `_generation_batch` (0 without one)."""
    return batch_rows_of(getattr(gen, "_generation_batch", None))


def decode_batch() -> int:
    """Decode concurrency from GMLX_DECODE_BATCH: a positive count as given,
    0 for the engine's own default (32), anything else 8."""
    n = _number("GMLX_DECODE_BATCH", DEFAULT_DECODE_BATCH)
    if n == 0 and os.environ.get("GMLX_DECODE_BATCH", "").strip():
        return UPSTREAM_DECODE_BATCH
    return n if n > 0 else DEFAULT_DECODE_BATCH


# -------------------------------------------------------------- the stamp

def row_bytes(ids) -> bytes:
    """A row's token ids as int32 bytes (the stamp's per-row format)."""
    return np.asarray([int(t) for t in ids], dtype=np.int32).tobytes()


def lcp_rows(rows: Sequence[bytes]) -> int:
    """Tokens every packed row starts with (0 for no rows or an empty one):
    the first mismatch of each row against the first, found on int32 views,
    so a partly equal token never counts."""
    if not rows:
        return 0
    views = [np.frombuffer(r, dtype=np.int32) for r in rows]
    n = min(v.size for v in views)
    first = views[0][:n]
    for v in views[1:]:
        diff = np.flatnonzero(first != v[:n])
        if diff.size:
            n = int(diff[0])
            first = first[:n]
    return n


@dataclass(frozen=True)
class PrefixStamp:
    """The shared prefix of a batch: P tokens common to every row, and each
    row's packed tokens (cache row order)."""
    P: int
    rows: Tuple[bytes, ...]

    @staticmethod
    def from_rows(rows) -> Optional["PrefixStamp"]:
        rows = tuple(rows)
        P = lcp_rows(rows)
        return PrefixStamp(P, rows) if P > 0 else None

    @staticmethod
    def read(cache) -> Optional["PrefixStamp"]:
        d = getattr(cache, "__dict__", {}).get(STAMP_ATTR) if cache is not None else None
        return None if d is None else PrefixStamp(int(d["P"]), tuple(d["tok"]))

    @staticmethod
    def store(cache, stamp: Optional["PrefixStamp"]):
        """Write `stamp` on `cache` in the interop format, or clear it."""
        if stamp is None:
            cache.__dict__.pop(STAMP_ATTR, None)
        else:
            setattr(cache, STAMP_ATTR, {"P": stamp.P, "tok": stamp.rows})

    def joined(self, other: Optional["PrefixStamp"]) -> Optional["PrefixStamp"]:
        """Stamp of this batch extended by `other`'s rows: the prefix both
        sides' shared prefixes have in common (None when there is none, or
        when `other` carries no stamp)."""
        if other is None or not self.rows or not other.rows:
            return None
        P = lcp_rows([self.rows[0][:4 * self.P], other.rows[0][:4 * other.P]])
        return PrefixStamp(P, self.rows + other.rows) if P > 0 else None

    def kept(self, keep) -> Optional["PrefixStamp"]:
        """Stamp after filtering rows by the boolean `keep` (None when no row
        is left); the shared prefix of the kept rows is at least P."""
        flags = keep.tolist() if hasattr(keep, "tolist") else list(keep)
        rows = tuple(r for r, k in zip(self.rows, flags) if k)
        return PrefixStamp(self.P, rows) if rows else None


def _hook_cache(cache):
    """Wrap a cache's extend / filter (once per cache object) so its stamp
    follows the rows: joined on extend, masked on filter."""
    for name, after in (("extend", _after_extend), ("filter", _after_filter)):
        method = getattr(cache, name, None)
        if method is None or getattr(method, HOOK_MARK, False):
            continue

        def hooked(arg, *args, _orig=method, _after=after, **kw):
            before = PrefixStamp.read(cache)
            out = _orig(arg, *args, **kw)
            _after(cache, before, arg)
            return out

        setattr(hooked, HOOK_MARK, True)
        setattr(cache, name, hooked)


def _after_extend(cache, before, other):
    PrefixStamp.store(cache, before.joined(PrefixStamp.read(other)) if before is not None else None)


def _after_filter(cache, before, keep):
    if before is not None:
        PrefixStamp.store(cache, before.kept(keep))


def _apply(cache, stamp: Optional[PrefixStamp]):
    PrefixStamp.store(cache, stamp)
    if stamp is not None:
        _hook_cache(cache)


def stamp_caches(caches, rows) -> bool:
    """Stamp every layer cache with the shared prefix of `rows` (packed
    tokens, cache row order).  False, and nothing stamped, when the rows
    share no token."""
    stamp = PrefixStamp.from_rows(rows)
    if stamp is None:
        return False
    for c in caches:
        _apply(c, stamp)
    _Counters.stamps += 1
    return True


def carry_stamp(src, dst):
    """Give a rebuilt cache object of the same rows its predecessor's stamp."""
    stamp = PrefixStamp.read(src)
    if stamp is not None and dst is not None:
        _apply(dst, stamp)


def rows_from_prompt_batch(pb):
    """Packed full prompt tokens per row of a newly formed prompt batch: the
    `_apc_meta[i]["full_input_ids"]` lists when the batch carries that meta
    (None if a row lacks them), else its `_input_ids` rows without their
    left / right padding; None when neither is there."""
    meta = getattr(pb, "_apc_meta", None)
    if meta:
        ids = [(m or {}).get("full_input_ids") for m in meta]
        return None if not all(ids) else [row_bytes(r) for r in ids]
    ids = getattr(pb, "_input_ids", None)
    left = getattr(pb, "_left_padding_per_row", None)
    if ids is None or left is None or len(getattr(ids, "shape", ())) != 2:
        return None
    right = list(getattr(pb, "_right_pad_per_row", None) or [])
    right += [0] * (len(left) - len(right))
    width = ids.shape[1]
    table = ids.tolist() if hasattr(ids, "tolist") else ids
    return [row_bytes(table[i][lp:width - rp]) for i, (lp, rp) in enumerate(zip(left, right))]


# ---------------------------------------------------------- row geometry

class _RowGeometry:
    """Per-cache memo of the left-padded layout: host pads for one
    `left_padding` object (batch changes rebind the attribute, so identity is
    the key), and the private-slab start table per (P, device)."""

    def __init__(self, lp):
        self.lp = lp
        self.pads = [int(v) for v in (lp.tolist() if hasattr(lp, "tolist") else lp)]
        self.tables = {}

    @staticmethod
    def of(cache) -> Optional["_RowGeometry"]:
        lp = getattr(cache, "left_padding", None)
        if lp is None:
            return None
        geo = cache.__dict__.get(GEOMETRY_ATTR)
        if geo is None or geo.lp is not lp:
            geo = _RowGeometry(lp)
            setattr(cache, GEOMETRY_ATTR, geo)
        return geo

    def slab(self, P: int, device, rows: Optional[int] = None):
        """(starts, c0): the private slab begins at column c0 = min(pads) + P
        and row b's private keys at starts[b] = pads[b] + P - c0 in it."""
        import torch
        pads = self.pads if rows is None else self.pads[:rows]
        key = (P, str(device), len(pads))
        hit = self.tables.get(key)
        if hit is None:
            c0 = min(pads) + P
            hit = (torch.tensor([p + P - c0 for p in pads], dtype=torch.int32, device=device), c0)
            self.tables[key] = hit
        return hit


def cache_pads(cache):
    """Host pads of a left-padded cache (memoised per `left_padding` object)."""
    geo = _RowGeometry.of(cache)
    return None if geo is None else geo.pads


def cascade_starts(cache, pads, P, device):
    """(starts int32 device tensor, c0) of a stamped cache's private slab."""
    return _RowGeometry.of(cache).slab(P, device, len(pads))


# ---------------------------------------------------------------- claims

def mask_claimable(mask, qL) -> bool:
    """Masks the cascade kernel reproduces: none at decode width; "causal";
    an explicit mask whose query axis has width qL (left pads plus the
    block's end-aligned causal part)."""
    if isinstance(mask, str):
        return mask == "causal"
    if mask is None:
        return qL == 1
    shape = getattr(mask, "shape", None)
    return shape is not None and len(shape) >= 2 and shape[-2] == qL


@dataclass
class _Call:
    """An attention call as the gates see it."""
    queries: object
    keys: object
    values: object
    cache: object
    mask: object
    sinks: object
    scale: float = 1.0
    quant: bool = False
    B: int = 0
    Hq: int = 0
    qL: int = 0
    D: int = 0
    Hkv: int = 0
    L: int = 0
    stamp: Optional[PrefixStamp] = None
    pads: Optional[list] = None

    @property
    def G(self):
        return self.Hq // self.Hkv if self.Hkv else 0


def _is_q8_cache(call) -> bool:
    """An 8-bit group-64 quantised cache presents K / V as (wire, scales,
    biases); at head dim 512 it is not claimed (the reference's gate,
    gmlx/cascade_sdpa.py:150-157), so such a call declines as 'quant-config'."""
    trio = lambda t: isinstance(t, (tuple, list)) and len(t) == 3  # noqa: E731
    return (trio(call.keys) and trio(call.values) and getattr(call.cache, "bits", None) == 8
            and getattr(call.cache, "group_size", None) == 64 and call.queries.shape[-1] != 512)


def _shape_call(call) -> Optional[str]:
    """Fill the call's dimensions; the decline reason when they cannot be read."""
    import torch
    call.quant = _is_q8_cache(call)
    if not call.quant and (isinstance(call.keys, (tuple, list)) or getattr(call.cache, "bits", None) is not None):
        return "quant-config"
    k = call.keys[0] if call.quant else call.keys
    v = call.values[0] if call.quant else call.values
    if not all(isinstance(t, torch.Tensor) for t in (call.queries, k, v)):
        return "not-tensors"
    if call.queries.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        return "rank"
    call.B, call.Hq, call.qL, call.D = call.queries.shape
    call.Hkv, call.L = k.shape[1], k.shape[2]
    want_last = call.D // 4 if call.quant else call.D          # four 8-bit values per uint32 word
    kv_dtype_ok = ((k.dtype in (torch.int32, getattr(torch, "uint32", torch.int32))
                    and call.keys[1].dtype == call.queries.dtype) if call.quant
                   else (k.dtype == call.queries.dtype and v.dtype == call.queries.dtype))
    if not (k.shape[0] == call.B and tuple(v.shape) == tuple(k.shape) and k.shape[3] == want_last
            and kv_dtype_ok and call.queries.dtype in (torch.float16, torch.bfloat16)):
        return "shape/dtype"
    return None


# Gates in order: (decline reason, test).  Each test sees a shaped call.
_GATES = (
    ("sinks", lambda c: c.sinks is None),
    ("single-row", lambda c: c.B > 1),
    ("width-q", lambda c: 1 <= c.qL <= 8),
    ("head-dim", lambda c: c.D in CASCADE_HEAD_DIMS),
    ("gqa", lambda c: c.Hkv >= 1 and c.Hq % c.Hkv == 0 and c.G <= 16),
    ("right-padding", lambda c: getattr(c.cache, "_right_padding", None) is None),
    ("mask", lambda c: mask_claimable(c.mask, c.qL)),
    ("width", lambda c: c.B * c.G * c.qL <= (32 if c.D == 512 else 64)),
    ("verify-width", lambda c: c.qL == 1 or c.G * ((c.qL + 1) // 2) <= 32),
    ("short-prefix", lambda c: c.stamp.P >= _number("GMLX_CASCADE_MIN_P", 1024)),
    ("pads", lambda c: c.pads is not None and len(c.pads) >= c.B),
    ("geometry", lambda c: (c.L - (min(c.pads[:c.B]) + c.stamp.P) >= c.qL
                            and max(c.pads[:c.B]) + c.stamp.P <= c.L - c.qL + 1)),
)


def _run_cascade(call):
    """The cascade op on views of the live cache buffers: the prefix is row
    0's copy at [pads[0], pads[0] + P), the private slab starts at c0."""
    from . import ops
    P = call.stamp.P
    starts, c0 = _RowGeometry.of(call.cache).slab(P, call.queries.device, call.B)
    p0 = call.pads[0]
    prefix = lambda t: t[0:1, :, p0:p0 + P]  # noqa: E731
    private = lambda t: t[:, :, c0:]  # noqa: E731
    if not call.quant:
        return ops.sdpa_decode_gqa_cascade(call.queries, prefix(call.keys), prefix(call.values),
                                           private(call.keys), private(call.values), call.scale, starts=starts)
    (kw, ks, kb), (vw, vs, vb) = call.keys, call.values
    return ops.sdpa_decode_gqa_cascade(
        call.queries, prefix(kw), prefix(vw), private(kw), private(vw), call.scale, starts=starts,
        k_shared_scales=prefix(ks), k_shared_biases=prefix(kb), v_shared_scales=prefix(vs),
        v_shared_biases=prefix(vb), k_priv_scales=private(ks), k_priv_biases=private(kb),
        v_priv_scales=private(vs), v_priv_biases=private(vb))


def cascade_claim(queries, keys, values, cache, scale, mask=None, sinks=None):
    """The cascade kernel's output for a stamped batched call that passes
    every gate, else None (the caller's stock attention runs).

    queries (B, Hq, qL, D); keys / values the cache's (B, Hkv, L, D) buffers
    (8-bit caches: (wire, scales, biases) triples), every row holding the
    shared prefix at [pads[b], pads[b] + P)."""
    stamp = PrefixStamp.read(cache) if cache is not None and hasattr(cache, "__dict__") else None
    if stamp is None:
        return _decline("no-stamp")
    call = _Call(queries, keys, values, cache, mask, sinks, scale, stamp=stamp)
    reason = _shape_call(call)
    if reason is not None:
        return _decline(reason)
    call.pads = cache_pads(cache)
    for reason, ok in _GATES:
        if not ok(call):
            return _decline(reason, B=call.B, qL=call.qL, D=call.D, G=call.G, P=stamp.P, L=call.L)
    from ._lib import KQLibraryError
    try:
        out = _run_cascade(call)
    except KQLibraryError:
        raise  # a missing library is a broken install, not a declined call
    except Exception as e:  # the route only declines
        return _decline("kernel", err=str(e)[:120])
    _Counters.claims += 1
    return out


# ----------------------------------------------------------------- routes

class _CascadeRoute:
    """A module's attention seam with the cascade claim in front: claimed
    calls run the cascade op, all others reach the original unchanged."""

    def __init__(self, orig):
        self.orig = orig

    def __call__(self, queries, keys, values, cache=None, scale=1.0, mask=None, sinks=None):
        out = cascade_claim(queries, keys, values, cache, scale, mask, sinks)
        if out is not None:
            return out
        return self.orig(queries, keys, values, cache=cache, scale=scale, mask=mask, sinks=sinks)


def make_route(orig):
    """Wrap an attention seam `orig(queries, keys, values, cache=None,
    scale=1.0, mask=None, sinks=None)` with the cascade claim."""
    return _CascadeRoute(orig)


def install_cascade_sdpa(modules) -> bool:
    """Put the cascade claim in front of each module's
    `scaled_dot_product_attention` seam (once; GMLX_CASCADE_SDPA=0 leaves
    them alone).  True when at least one module has the seam."""
    if not cascade_enabled():
        return False
    found = False
    for mod in modules:
        seam = getattr(mod, "scaled_dot_product_attention", None)
        if seam is None:
            continue
        found = True
        if not isinstance(seam, _CascadeRoute):
            mod.scaled_dot_product_attention = _CascadeRoute(seam)
    return found


def left_padded_attention(queries, keys, values, *, cache, scale, mask=None):
    """A left-padded batched decode call: the cascade claim first (B > 1,
    qL 1, GMLX_CASCADE_SDPA on), then the ragged kernel; None when neither
    takes it.  Quantised caches, non-4-D tensors and unpadded batches
    decline at once."""
    from . import ops
    from ._lib import KQLibraryError
    if getattr(cache, "bits", None) is not None:
        return None
    if getattr(queries, "dim", lambda: 0)() != 4 or getattr(keys, "dim", lambda: 0)() != 4:
        return None
    pads = getattr(cache, "__dict__", {}).get("_qwen3_5_decode_left_padding") or cache_pads(cache)
    if not pads or max(pads) <= 0:
        return None
    if queries.shape[0] > 1 and queries.shape[2] == 1 and cascade_enabled():
        out = cascade_claim(queries, keys, values, cache, scale, None, None)
        if out is not None:
            return out
    try:
        return ops.ragged_decode_attention(queries, keys, values, list(pads), scale)
    except KQLibraryError:
        raise
    except Exception as e:
        return _decline("ragged", err=str(e)[:120])


# ------------------------------------------------ stamping at batch formation

class _StampingInit:
    """A prompt batch constructor that stamps the new batch's caches with
    their rows' shared prefix (stamping never breaks batch formation)."""

    def __init__(self, orig):
        self.orig = orig

    def __get__(self, obj, owner=None):
        if obj is None:
            return self
        return lambda *a, **kw: self(obj, *a, **kw)

    def __call__(self, batch, *args, **kw):
        self.orig(batch, *args, **kw)
        try:
            caches = getattr(batch, "prompt_cache", None)
            rows = rows_from_prompt_batch(batch) if caches else None
            if rows:
                stamp_caches(caches, rows)
            else:
                _decline("stamp-no-rows")
        except Exception as e:
            _decline("stamp", err=str(e)[:120])


class _StampingExtend:
    """The engine's cache-list merge with the stamps joined per layer."""

    def __init__(self, orig):
        self.orig = orig

    def __call__(self, a, b):
        sides = [(PrefixStamp.read(ca), PrefixStamp.read(cb)) for ca, cb in zip(a, b)]
        out = self.orig(a, b)
        for cache, (sa, sb) in zip(out, sides):
            _apply(cache, sa.joined(sb) if sa is not None else None)
        return out


def install_cascade_stamp(engine_module) -> bool:
    """Stamp batches as a serving engine module forms them: its
    `PromptProcessingBatch.__init__` and `_extend_cache` (the two hooks the
    reference patches).  Idempotent; GMLX_CASCADE_SDPA=0 disables it."""
    if not cascade_enabled():
        return False
    ppb = getattr(engine_module, "PromptProcessingBatch", None)
    ext = getattr(engine_module, "_extend_cache", None)
    if ppb is None or ext is None:
        return False
    if not isinstance(ppb.__dict__.get("__init__"), _StampingInit):
        ppb.__init__ = _StampingInit(ppb.__init__)
    if not isinstance(ext, _StampingExtend):
        engine_module._extend_cache = _StampingExtend(ext)
    return True
