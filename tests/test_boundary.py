"""CPU tests of the drop-in boundary: library exports, host-side validation.

No kernel is launched here (no GPU in the CPU suite): the library is loaded
with ctypes and its exported symbols are compared with include/nsq_hip.h; the
Python layer's argument checks are exercised with CPU tensors, which must be
rejected loudly rather than computed on the CPU.
"""

import os
import re
import subprocess

import pytest
import torch

from nvsubquadratic_amd import _lib
from nvsubquadratic_amd import fftconv_hip as F


ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nsq_hip.h")


def _header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nsq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_what_python_binds():
    assert _header_functions() == _lib.library_exports()


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="libnsq_hip.so not built")
def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True)
    exported = set(re.findall(r"\bT (nsq_[a-z0-9_]+)$", out.stdout, flags=re.M))
    missing = [f for f in _header_functions() if f not in exported]
    assert not missing, missing


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="libnsq_hip.so not built")
def test_library_loads_and_reports_abi():
    lib = _lib.get_lib()
    assert lib.nsq_abi_version() == _lib.ABI_VERSION
    assert isinstance(lib.nsq_last_error(), bytes)


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="libnsq_hip.so not built")
def test_workspace_query_needs_no_gpu():
    lib = _lib.get_lib()
    # fused plan (F <= 16384): no workspace
    assert lib.nsq_fftconv1d_causal_workspace_bytes(2, 128, 4096, 4096, 0) == 0
    # 4-step plan at config 3: one complex64 row per signal
    n = 1 << 18
    assert lib.nsq_fftconv1d_causal_workspace_bytes(1, 4096, 262144, 262144, 0) == (4096 + 4096) * n * 8
    assert lib.nsq_fftconv1d_causal_workspace_bytes(1, 4096, 262144, 262144, 1) == (2 * 4096 + 4096) * n * 8
    # K > L+1 on the 4-step plan (FFT length pow2(3L)): one more block of B*H*N complex values for the wrap copy
    nf = 1 << 16  # L = 2^15: F = 2^17, N = 2^16
    assert lib.nsq_fftconv1d_causal_workspace_bytes(2, 3, 32768, 65536, 0) == (6 + 3 + 6) * nf * 8
    assert lib.nsq_fftconv1d_causal_workspace_bytes(2, 3, 32768, 65536, 1) == (2 * 6 + 3 + 6) * nf * 8


def test_per_sample_film_kernel_batch_validated():
    """tests/ops/test_fftconv_custom_1d.py:231-239 checks that the reference's native wrapper rejects [B, H, K];
    this backend accepts it (the torch path's semantics, fftconv.py:546-600) and rejects only a kernel batch that
    is neither 1 nor B, in Python (AssertionError, as fftconv.py:571-574) and in the C ABI (before the device)."""
    x = torch.randn(2, 32, 128)
    with pytest.raises(AssertionError, match="Leading dimension must be 1 or batch_size"):
        F.causal_fftconv1d_bhl(x, torch.randn(3, 32, 5))
    lib = _lib.get_lib()
    dummy = 16
    rc = lib.nsq_fftconv1d_causal_film_fwd(dummy, dummy, None, dummy, _lib.NSQ_DTYPE[torch.float32], 2, 32, 128, 5,
                                           3, None, 0, None)
    assert rc == 1 and b"kernel batch" in lib.nsq_last_error()
    # per-sample filters size the 4-step workspace with B*H filter rows
    shared = lib.nsq_fftconv1d_causal_workspace_bytes(2, 4, 65536, 65536, 1)
    film = lib.nsq_fftconv1d_causal_film_workspace_bytes(2, 4, 65536, 65536, 2, 1)
    assert film - shared == 4 * (shared // (2 * 2 * 4 + 4))


def test_kernel_longer_than_two_l_rejected():
    with pytest.raises(ValueError, match="2 \\* seq_len"):
        F.causal_fftconv1d_bhl(torch.randn(1, 2, 8), torch.randn(1, 2, 17))


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="libnsq_hip.so not built")
def test_cpu_tensors_fail_loudly_no_cpu_fallback():
    with pytest.raises(_lib.HipLibraryError, match="no CPU fallback"):
        F.causal_fftconv1d_bhl(torch.randn(1, 2, 8), torch.randn(1, 2, 3))


def test_missing_library_raises_at_call_time(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "nope.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(_lib.HipLibraryError, match="not found"):
        _lib.get_lib()


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="libnsq_hip.so not built")
def test_nd_plan_uses_the_reference_fft_sizes_where_smaller(monkeypatch):
    """Zero-padded 2D / 3D axes run at the reference's F_d = S_d + ceil(K_d/2) rounded to 48 / 96 / 192 when that
    spectrum is smaller than the power-of-two one (ops/fftconv.py:699-702, 774-778); NSQ_ND_R3=0 selects the
    power-of-two plan.  Read back through the workspace size: (B*H + H) spectrum blocks of F0 F1 (F2/2 + 1)."""
    lib = _lib.get_lib()

    def fwd_bytes(xs, ks):
        S, K = _lib.i64_array(xs[2:]), _lib.i64_array(ks)
        return lib.nsq_fftconv_nd_workspace_bytes(3, xs[0], xs[1], S, K, 1, _lib.NSQ_DIR_FWD)

    def blocks(xs, f0, f1, f2):
        return (xs[0] * xs[1] + xs[1]) * f0 * f1 * (f2 // 2 + 1) * 8

    cfg5 = ((2, 128, 64, 64, 64), (64, 64, 64))
    assert fwd_bytes(*cfg5) == blocks(cfg5[0], 96, 96, 96)
    assert fwd_bytes((1, 2, 128, 32, 32), (128, 32, 32)) == blocks((1, 2), 192, 48, 48)
    assert fwd_bytes((2, 3, 33, 45, 27), (29, 7, 41)) == blocks((2, 3), 48, 96, 48)
    # power of two where it is smaller: need 11 -> 16 on axis 0 (48 would be larger)
    assert fwd_bytes((1, 2, 9, 64, 64), (4, 64, 64)) == blocks((1, 2), 16, 128, 128)
    # an axis past 96 (axes 1, 2) keeps the power-of-two plan: 6+3 -> 16, 100+11 -> 128, 50+14 -> 64
    assert fwd_bytes((1, 2, 6, 100, 50), (5, 21, 27)) == blocks((1, 2), 16, 128, 64)
    # 2D: config 4's 128^2 with K = 128 at 192^2 (rows of 97 bins) instead of 256^2 (128 packed bins)
    S2, K2 = _lib.i64_array([128, 128]), _lib.i64_array([128, 128])
    assert lib.nsq_fftconv_nd_workspace_bytes(2, 16, 384, S2, K2, 1, _lib.NSQ_DIR_FWD) == (16 * 384 + 384) * 192 * 97 * 8
    monkeypatch.setenv("NSQ_ND_R3", "0")
    assert fwd_bytes(*cfg5) == blocks(cfg5[0], 128, 128, 128)
    assert lib.nsq_fftconv_nd_workspace_bytes(2, 16, 384, S2, K2, 1, _lib.NSQ_DIR_FWD) == (16 * 384 + 384) * 256 * 128 * 8
    # periodic axes keep F_d = S_d
    S, K = _lib.i64_array([64, 64, 64]), _lib.i64_array([64, 64, 64])
    monkeypatch.delenv("NSQ_ND_R3")
    assert lib.nsq_mixed_fftconv_nd_workspace_bytes(3, 2, 128, S, K, 1, 1, _lib.NSQ_DIR_FWD) == blocks(
        cfg5[0], 64, 128, 128)


def test_nd_spectrum_block_over_2gib_rejected():
    """The 2D/3D column passes address one spectrum block with 32-bit byte
    offsets; a block of 2 GiB or more (F = 1024^3: 1024*1024*513 complex) must be
    refused before any launch (validation runs before the device is touched)."""
    lib = _lib.get_lib()
    dummy = 16  # non-null; never dereferenced when validation fails
    S, K = _lib.i64_array([1000, 1000, 1000]), _lib.i64_array([3, 3, 3])
    rc = lib.nsq_fftconv_nd_fwd(3, dummy, dummy, None, dummy, _lib.NSQ_DTYPE[torch.float32], 1, 1, S, K, 1, dummy,
                                1 << 40, None)
    assert rc == 2  # NSQ_ERR_UNSUPPORTED
    assert b"2 GiB" in lib.nsq_last_error()


def test_periodic_lengths_validated_before_launch():
    """Circular / mixed entry points refuse non-power-of-two or out-of-range
    periodic lengths (NSQ_ERR_UNSUPPORTED) and periodic kernels longer than the
    axis (NSQ_ERR_INVALID_ARGUMENT) before the device is touched."""
    lib = _lib.get_lib()
    dummy = 16
    f32 = _lib.NSQ_DTYPE[torch.float32]
    assert lib.nsq_circular_fftconv1d_fwd(dummy, dummy, None, dummy, f32, 1, 1, 48, 5, 1, None) == 2
    assert b"power" in lib.nsq_last_error()
    assert lib.nsq_circular_fftconv1d_fwd(dummy, dummy, None, dummy, f32, 1, 1, 32768, 5, 1, None) == 2
    assert lib.nsq_circular_fftconv1d_fwd(dummy, dummy, None, dummy, f32, 1, 1, 64, 65, 1, None) == 1
    assert lib.nsq_circular_fftconv1d_bwd(dummy, dummy, dummy, None, dummy, dummy, None, f32, 2, 1, 64, 5, 3,
                                          None) == 1  # kernel batch neither 1 nor B
    S, K = _lib.i64_array([12, 16]), _lib.i64_array([3, 3])
    assert lib.nsq_mixed_fftconv_nd_workspace_bytes(2, 1, 1, S, K, 1, 0b01, 0) == 0
    rc = lib.nsq_mixed_fftconv_nd_fwd(2, dummy, dummy, None, dummy, f32, 1, 1, S, K, 1, 0b01, dummy, 1 << 40, None)
    assert rc == 2 and b"periodic axis 0" in lib.nsq_last_error()
    # axis 0 zero-padded is fine at 12; axis 1 periodic at 16 with K = 17 is not
    S, K = _lib.i64_array([12, 16]), _lib.i64_array([3, 17])
    rc = lib.nsq_mixed_fftconv_nd_fwd(2, dummy, dummy, None, dummy, f32, 1, 1, S, K, 1, 0b10, dummy, 1 << 40, None)
    assert rc == 1
    rc = lib.nsq_mixed_fftconv_nd_fwd(2, dummy, dummy, None, dummy, f32, 1, 1, S, K, 1, 0b100, dummy, 1 << 40, None)
    assert rc == 1 and b"periodic mask" in lib.nsq_last_error()
    S, K = _lib.i64_array([12, 64]), _lib.i64_array([3, 64])
    spec_zero = lib.nsq_fftconv_nd_workspace_bytes(2, 1, 1, S, K, 1, 0)
    spec_mixed = lib.nsq_mixed_fftconv_nd_workspace_bytes(2, 1, 1, S, K, 1, 0b10, 0)
    assert 0 < 2 * spec_mixed == spec_zero  # the periodic axis is not padded: F1 = 64 instead of 128
    # short periods run on their periodic extension at length 16 (accepted, not refused)
    S, K = _lib.i64_array([8, 4]), _lib.i64_array([3, 4])
    assert lib.nsq_mixed_fftconv_nd_workspace_bytes(2, 1, 1, S, K, 1, 0b11, 0) > 0


def test_noalloc_scratch_size_matches_header():
    m = re.search(r"#define NSQ_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", open(HEADER).read())
    assert m and int(m.group(1)) << int(m.group(2)) == _lib.NSQ_NOALLOC_SCRATCH_BYTES


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="libnsq_hip.so not built")
def test_noalloc_backward_refuses_oversize_scratch_on_the_host():
    """A shape whose scratch exceeds the fixed device buffer is refused before anything touches the GPU."""
    lib = _lib.get_lib()
    B, C, L, K = 8, 8192, 1 << 20, 16
    assert lib.nsq_causal_conv1d_bwd_workspace_bytes(B, C, L, K, 0) > _lib.NSQ_NOALLOC_SCRATCH_BYTES
    fake = 1 << 20  # never dereferenced: the call returns before any launch
    rc = lib.nsq_causal_conv1d_bwd_noalloc(fake, fake, fake, None, fake, fake, None, 0, 0, B, C, L, K, None)
    assert rc == 2  # NSQ_ERR_UNSUPPORTED
    assert b"scratch" in lib.nsq_last_error()


_OPS = ["causal_fftconv1d", "fftconv_nd", "shifted_fftconv1d", "causal_conv1d", "b2b_causal_conv1d",
        "gated_causal_fftconv1d", "gated_fftconv_nd", "gated_channel_rmsnorm", "gated_channel_layernorm",
        "gated_channel_groupnorm", "channel_l2norm"]


def test_every_hip_op_is_a_registered_custom_op():
    """Each op and its backward are torch.library custom ops (traceable by torch.compile)."""
    import nvsubquadratic_amd.causal_conv1d_hip  # noqa: F401
    import nvsubquadratic_amd.gated_fftconv_hip  # noqa: F401
    import nvsubquadratic_amd.norm_hip  # noqa: F401

    for name in _OPS:
        for n in (name, name + "_backward"):
            schema = str(getattr(torch.ops.nsq_hip, n).default._schema)
            assert schema.startswith(f"nsq_hip::{n}(")


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="libnsq_hip.so not built")
def test_fake_implementations_propagate_shapes_without_a_gpu():
    """The fake (meta) implementations give the real ops' output shapes and the forward-state size the C ABI
    reports, with no device code involved."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    lib = _lib.get_lib()
    with FakeTensorMode():
        x = torch.empty(2, 4, 50000)
        k = torch.empty(4, 50000)
        s = torch.empty(4)
        y, state = torch.ops.nsq_hip.causal_fftconv1d(x, k, s, 1, True)
        assert y.shape == x.shape and state.dtype == torch.uint8
        assert state.numel() == lib.nsq_fftconv1d_causal_workspace_bytes(2, 4, 50000, 50000, _lib.NSQ_DIR_BWD)
        gx, gk, gs = torch.ops.nsq_hip.causal_fftconv1d_backward(x, x, k, s, state, 1)
        assert gx.shape == x.shape and gk.shape == k.shape and gs.shape == (4,)
        x2 = torch.empty(2, 3, 16, 12)
        y2, st2 = torch.ops.nsq_hip.fftconv_nd(x2, torch.empty(3, 5, 7), None, 1, 0, False)
        assert y2.shape == x2.shape and st2.numel() == 0
        yb = torch.ops.nsq_hip.b2b_causal_conv1d(torch.empty(2, 12, 64), torch.empty(12, 3), torch.empty(4, 9), None)
        assert yb.shape == (2, 4, 64)
        import nvsubquadratic_amd.norm_hip  # noqa: F401

        yn = torch.empty(3, 12, 40)
        gn, mean, rstd = torch.ops.nsq_hip.gated_channel_groupnorm(yn, yn, torch.empty(12), None, 4, 1e-5, 1)
        assert gn.shape == yn.shape and mean.shape == (3, 4) and rstd.shape == (3, 4)
        dyn, dvn, dwn, dbn = torch.ops.nsq_hip.gated_channel_groupnorm_backward(yn, yn, yn, torch.empty(12), mean,
                                                                                rstd, False, 1)
        assert dyn.shape == yn.shape and dvn.shape == yn.shape and dwn.shape == (12,) and dbn.numel() == 0


def test_transpose_launch_limits_and_fallback():
    """The batched transpose takes any row count (row tiles on grid.x) but at most 65535 batches and 65535
    column tiles; beyond that the library refuses before any launch and the layout helper falls back to
    ``Tensor.contiguous``."""
    from nvsubquadratic_amd.layout import transpose_fits

    assert transpose_fits(65535, 65535 * 64)
    assert not transpose_fits(65536, 8)
    assert not transpose_fits(1, 65535 * 64 + 1)
    assert transpose_fits(1, 8)  # any R: the row tiles are not limited to 65535
    if not os.path.exists(_lib.LIB_PATH):
        return
    lib = _lib.get_lib()
    fake_src, fake_dst = 1 << 20, 2 << 20  # argument checks run before any HIP call; nothing is dereferenced
    assert lib.nsq_batched_transpose(fake_src, fake_dst, 2, 1, 64, 65535 * 64 + 1, None) != 0
    assert b"exceed the launch grid" in lib.nsq_last_error()
    assert lib.nsq_batched_transpose(fake_src, fake_dst, 2, 65536, 64, 8, None) != 0
    assert lib.nsq_batched_transpose(fake_src, fake_dst, 3, 1, 64, 8, None) != 0


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="libnsq_hip.so not built")
def test_channel_norm_backward_limit_raised_before_forward():
    """3536 < C <= 7781: the forward would run, its backward cannot; with a gradient wanted the call refuses up
    front (host-side query, no launch), without one it goes on to the device check."""
    from nvsubquadratic_amd import norm_hip as N

    lib = _lib.get_lib()
    assert lib.nsq_channel_rmsnorm_bwd_workspace_bytes(2, 3536, 64) > 0
    assert lib.nsq_channel_rmsnorm_bwd_workspace_bytes(2, 3537, 64) == 0
    y = torch.randn(2, 4000, 8, requires_grad=True)
    w = torch.ones(4000)
    with pytest.raises(NotImplementedError, match="C <= 3536"):
        N.gated_channel_rmsnorm(y, None, w)
    with torch.no_grad(), pytest.raises(_lib.HipLibraryError):
        N.gated_channel_rmsnorm(y, None, w)  # forward-only: passes the limit, then refuses CPU tensors
