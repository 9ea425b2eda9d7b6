"""The allocation-free decode attention entry point, kq_sdpa_decode_gqa_noalloc
(no counterpart in the reference: for callers that cannot allocate), against
kq_sdpa_decode_gqa with a caller workspace, both through the C ABI: outputs
bitwise equal (the same kernels and split plan) on two calls in a row, the
second smaller than the first, and the first also within tolerance of the
fp64 reference; a request past the scratch limit is refused before any
launch."""
import numpy as np
import pytest

from helpers import TOL, attention_ref
from oracle import kquant as okq

pytestmark = pytest.mark.gpu


def _inputs(torch, rng, B, Hq, Hkv, D, L):
    k = torch.from_numpy(rng.normal(0, 1, size=(B, Hkv, L, D)).astype(np.float16)).cuda()
    v = torch.from_numpy(rng.normal(0, 1, size=(B, Hkv, L, D)).astype(np.float16)).cuda()
    q = torch.from_numpy(rng.normal(0, 1, size=(B, Hq, D)).astype(np.float16)).cuda()
    starts = torch.from_numpy(rng.integers(0, L // 2, size=B).astype(np.int32)).cuda()
    return q, k, v, starts


def _call(torch, L_, q, k, v, starts, Hkv, ws=None):
    from gmlx_amd import _lib
    B, Hq, D = q.shape
    L = k.shape[2]
    out = torch.full_like(q, float("nan"))
    stream = torch.cuda.current_stream().cuda_stream
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), L, starts.data_ptr(), B, Hq, Hkv,
            D, D ** -0.5, _lib.DTYPE_F16, out.data_ptr())
    if ws is None:
        rc = L_.kq_sdpa_decode_gqa_noalloc(*args, stream)
    else:
        rc = L_.kq_sdpa_decode_gqa(*args, ws.data_ptr(), ws.numel(), stream)
    assert rc == 0, rc
    torch.cuda.synchronize()
    return out


def test_noalloc_matches_workspace_entry_twice():
    import torch
    from gmlx_amd import _lib
    L_ = _lib.lib()
    rng = np.random.default_rng(77)
    for B, Hq, Hkv, D, L in [(6, 16, 4, 128, 3000), (3, 8, 2, 64, 700)]:
        q, k, v, starts = _inputs(torch, rng, B, Hq, Hkv, D, L)
        need = L_.kq_sdpa_workspace_bytes(B, Hq, Hkv, D, L)
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        want = _call(torch, L_, q, k, v, starts, Hkv, ws).cpu().numpy()
        got = _call(torch, L_, q, k, v, starts, Hkv).cpu().numpy()
        assert np.array_equal(got.view(np.uint16), want.view(np.uint16)), (B, Hq, Hkv, D, L)
        if B == 6:
            qn, kn, vn, st = q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(), starts.cpu().numpy()
            ref = np.stack([attention_ref(qn[b], kn[b, :, st[b]:], vn[b, :, st[b]:], D ** -0.5) for b in range(B)])
            assert okq.max_rel(got.astype(np.float32), ref) <= TOL


def test_noalloc_refuses_requests_past_its_scratch():
    from gmlx_amd import _lib
    L_ = _lib.lib()
    B, Hq, Hkv, D, L = 64, 64, 8, 256, 200000
    assert L_.kq_sdpa_workspace_bytes(B, Hq, Hkv, D, L) > _lib.SDPA_NOALLOC_SCRATCH_BYTES
    rc = L_.kq_sdpa_decode_gqa_noalloc(None, None, None, Hkv * L * D, L * D, L, None, B, Hq, Hkv, D, 0.0625,
                                       _lib.DTYPE_F16, None, None)
    assert rc == _lib.KQ_ERR_WORKSPACE_TOO_SMALL
