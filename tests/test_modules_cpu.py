"""Construction checks of the module drop-ins and the fft_backend dispatch (CPU)."""

import pytest
import torch

from nvsubquadratic_amd import dispatch
from nvsubquadratic_amd.modules import HipCausalConv1d


def test_rejects_non_depthwise():
    with pytest.raises(ValueError, match="depthwise-only"):
        HipCausalConv1d(in_channels=16, out_channels=16, kernel_size=3, groups=4)


def test_rejects_in_neq_out():
    with pytest.raises(ValueError, match="depthwise-only"):
        HipCausalConv1d(in_channels=16, out_channels=32, kernel_size=3, groups=16)


def test_rejects_invalid_activation():
    with pytest.raises(ValueError, match="activation"):
        HipCausalConv1d(in_channels=16, out_channels=16, kernel_size=3, groups=16, activation="relu")


def test_is_nn_conv1d_subclass_with_reference_state_dict_layout():
    m = HipCausalConv1d(in_channels=16, out_channels=16, kernel_size=3, groups=16, bias=True)
    assert isinstance(m, torch.nn.Conv1d)
    sd = m.state_dict()
    assert sd["weight"].shape == (16, 1, 3) and sd["bias"].shape == (16,)


def test_backend_name_validation():
    dispatch.validate_fft_backend("hip")
    with pytest.raises(AssertionError, match="Invalid fft_backend"):
        dispatch.validate_fft_backend("cufft")


def test_hip_constraints_mirror_reference_messages():
    with pytest.raises(AssertionError, match="does not support causal"):
        dispatch.validate_hip_backend(2, True, "zero")
    with pytest.raises(AssertionError, match="does not support causal"):
        dispatch.validate_hip_backend(3, True, ["zero", "circular", "zero"])
    with pytest.raises(AssertionError, match="not supported with fft_padding='circular'"):
        dispatch.validate_hip_backend(2, False, "circular", use_chunked_fftconv=True)
    with pytest.raises(AssertionError, match="data_dim"):
        dispatch.validate_hip_backend(4, False, "zero")
    dispatch.validate_hip_backend(1, False, "zero")
    dispatch.validate_hip_backend(1, False, "zero", use_chunked_fftconv=True)
    dispatch.validate_hip_backend(1, False, "circular")
    dispatch.validate_hip_backend(1, False, ["circular"])
    dispatch.validate_hip_backend(3, False, "circular")
    dispatch.validate_hip_backend(2, False, ["zero", "circular"], use_chunked_fftconv=True)


def test_resolve_periodic_mirrors_reference_forms_and_errors():
    assert dispatch.resolve_periodic("zero", 3) == (False, False, False)
    assert dispatch.resolve_periodic(" Circular ", 2) == (True, True)
    assert dispatch.resolve_periodic(["circular", "ZERO"], 2) == (True, False)
    for bad, msg in ((True, "True/False"), ("circular, zero", "comma-separated"), ((True, False), "booleans"),
                     (["circular"], "length data_dim"), (["periodic", "zero"], "Invalid padding mode"), (3, "single")):
        with pytest.raises(ValueError, match=msg):
            dispatch.resolve_periodic(bad, 2)


def test_hip_fn_selection():
    from nvsubquadratic_amd import fftconv_hip as F

    assert dispatch.hip_fftconv_fns(1, True) == (F.causal_fftconv1d_bhl_w_reshape, F.causal_fftconv1d_bhl)
    assert dispatch.hip_fftconv_fns(1, True, use_chunked_fftconv=True) == (
        F.causal_fftconv1d_bhl_w_reshape_chunked, F.causal_fftconv1d_bhl_chunked)
    # non-causal 1D: FFT_FUNCTIONS["zero"][1] (ckconv_nd.py:208-211) and its chunked table entry
    assert dispatch.hip_fftconv_fns(1, False, "zero") == (F.fftconv1d_bhl_w_reshape, F.fftconv1d_bhl)
    assert dispatch.hip_fftconv_fns(1, False, "zero", use_chunked_fftconv=True) == (
        F.fftconv1d_bhl_w_reshape_chunked, F.fftconv1d_bhl_chunked)


def test_hip_fn_selection_2d_3d():
    from nvsubquadratic_amd import fftconv_hip as F

    assert dispatch.hip_fftconv_fns(2, False) == (F.fftconv2d_bhl_w_reshape, F.fftconv2d_bhl)
    assert dispatch.hip_fftconv_fns(3, False, use_chunked_fftconv=True) == (
        F.fftconv3d_bhl_w_reshape_chunked, F.fftconv3d_bhl_chunked)


def test_hip_fn_selection_circular_and_mixed():
    from nvsubquadratic_amd import circular_fftconv_hip as C
    from nvsubquadratic_amd import mixed_fftconv_hip as M

    assert dispatch.hip_fftconv_fns(1, False, "circular") == (C.circular_fftconv1d_fp32_bhl_w_reshape,
                                                              C.circular_fftconv1d_fp32_bhl)
    assert dispatch.hip_fftconv_fns(3, False, "circular") == (C.circular_fftconv3d_fp32_bhl_w_reshape,
                                                              C.circular_fftconv3d_fp32_bhl)
    blh, bhl = dispatch.hip_fftconv_fns(2, False, ["circular", "zero"])
    assert bhl.op is M.mixed_fftconv2d_fp32_bhl and bhl.periodic == (True, False)
    assert blh.op is M.mixed_fftconv2d_fp32_bhl_w_reshape
    blh, bhl = dispatch.hip_fftconv_fns(3, False, ["zero", "circular", "zero"], use_chunked_fftconv=True)
    assert bhl.op is M.mixed_fftconv3d_fp32_bhl_chunked and bhl.periodic == (False, True, False)
