"""The allocation-free direct-conv backward (nsq_causal_conv1d_bwd_noalloc) against the
workspace entry point it mirrors (nsq_causal_conv1d_bwd), both called through the C ABI.

Both run the same kernels in the same order, so the outputs must agree bitwise.  Two calls
in a row on the shared device scratch, the second with a smaller input, show that nothing
from the first call leaks into the second; shapes cover the register path (K <= 16, only
weight / bias partials in scratch) and the matrix-core path with silu (K > 16, where the
pre-activation gradient lives in scratch too).  A shape whose scratch exceeds the fixed
buffer is refused on the host with NSQ_ERR_UNSUPPORTED.
"""

import pytest
import torch

from nvsubquadratic_amd import _lib


pytestmark = pytest.mark.gpu

ACT = {"identity": 0, "silu": 1}


def _inputs(B, C, L, K, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(B, C, L, device="cuda", generator=g).to(dtype)
    gy = torch.randn(B, C, L, device="cuda", generator=g).to(dtype)
    w = torch.randn(C, K, device="cuda", generator=g) / K ** 0.5
    b = torch.randn(C, device="cuda", generator=g)
    return x, gy, w, b


def _bwd_workspace(lib, x, gy, w, b, act):
    B, C, L = x.shape
    K = w.shape[1]
    gx, gw, gb = torch.empty_like(x), torch.empty_like(w), torch.empty_like(b)
    need = lib.nsq_causal_conv1d_bwd_workspace_bytes(B, C, L, K, act)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    _lib.check(lib.nsq_causal_conv1d_bwd(
        gy.data_ptr(), x.data_ptr(), w.data_ptr(), b.data_ptr(), gx.data_ptr(), gw.data_ptr(), gb.data_ptr(),
        _lib.dtype_code(x.dtype), act, B, C, L, K, ws.data_ptr(), need, _lib.stream_ptr(x.device)))
    return gx, gw, gb


def _bwd_noalloc(lib, x, gy, w, b, act):
    B, C, L = x.shape
    K = w.shape[1]
    gx, gw, gb = torch.empty_like(x), torch.empty_like(w), torch.empty_like(b)
    _lib.check(lib.nsq_causal_conv1d_bwd_noalloc(
        gy.data_ptr(), x.data_ptr(), w.data_ptr(), b.data_ptr(), gx.data_ptr(), gw.data_ptr(), gb.data_ptr(),
        _lib.dtype_code(x.dtype), act, B, C, L, K, _lib.stream_ptr(x.device)))
    return gx, gw, gb


@pytest.mark.parametrize("first,second", [
    ((4, 256, 8192, 4, "silu", torch.bfloat16), (2, 64, 1000, 3, "identity", torch.bfloat16)),
    ((2, 128, 4096, 64, "silu", torch.float32), (1, 16, 777, 17, "silu", torch.float32)),
    ((3, 96, 5000, 128, "identity", torch.float16), (2, 8, 300, 7, "silu", torch.float16)),
])
def test_noalloc_backward_matches_workspace_entry_point_twice(first, second):
    lib = _lib.get_lib()
    for seed, (B, C, L, K, act, dtype) in enumerate((first, second)):
        print(f"noalloc case B={B} C={C} L={L} K={K} {act} {dtype}", flush=True)
        need = lib.nsq_causal_conv1d_bwd_workspace_bytes(B, C, L, K, ACT[act])
        assert 0 < need <= _lib.NSQ_NOALLOC_SCRATCH_BYTES
        x, gy, w, b = _inputs(B, C, L, K, dtype, seed)
        ref = _bwd_workspace(lib, x, gy, w, b, ACT[act])
        got = _bwd_noalloc(lib, x, gy, w, b, ACT[act])
        torch.cuda.synchronize()
        for r, o in zip(ref, got):
            assert torch.equal(r, o)


def test_noalloc_refuses_shapes_beyond_its_scratch():
    lib = _lib.get_lib()
    B, C, L, K = 8, 8192, 1 << 20, 16
    need = lib.nsq_causal_conv1d_bwd_workspace_bytes(B, C, L, K, ACT["identity"])
    assert need > _lib.NSQ_NOALLOC_SCRATCH_BYTES
    x = torch.empty(1, device="cuda")  # never read: the call is refused before any launch
    rc = lib.nsq_causal_conv1d_bwd_noalloc(x.data_ptr(), x.data_ptr(), x.data_ptr(), None, x.data_ptr(),
                                          x.data_ptr(), None, 0, 0, B, C, L, K, _lib.stream_ptr(x.device))
    assert rc == 2  # NSQ_ERR_UNSUPPORTED
    assert b"scratch" in lib.nsq_last_error()
