"""RMSNorm forward (nf4s_rmsnorm_fwd) against the oracle's rms_norm_fwd
(doublepass/src/math.rs:36-59) on the same fp32 inputs.  The device sums the
squares as a tree, the reference in index order: the device's rms is checked
against the exact (fp64) rms to 2e-6 and against the oracle's to the oracle's
own distance from it; given the device's rms, y = bf16(x / rms * w) is
checked bit for bit, and it is never more than one bf16 ulp from the
oracle's y."""
import numpy as np
import pytest
import torch

import oracle
from aethelstream_amd import norm

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,d", [(1, 4), (7, 100), (130, 4096), (64, 8192), (5, 16384), (3, 32768)])
def test_rmsnorm_vs_oracle(m, d):
    x = oracle.gen_normal(70 + d, m * d, 1.0).reshape(m, d)
    x[0, : d // 2] *= 50.0                      # a row with a wide range
    w = (1.0 + oracle.gen_normal(71, d, 0.1)).astype(np.float32)
    y_ref, _, rms_ref = oracle.rmsnorm_fwd(x, w)
    y, rms = norm.rms_norm_fwd(torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda())
    torch.cuda.synchronize()
    rms_g = rms.cpu().numpy()
    # The tree sum is within fp32 rounding of the exact rms; the reference's
    # index-order sum can drift further (6e-5 on the wide-range row at
    # d = 32768), so the oracle comparison allows the oracle's own error.
    r64 = np.sqrt((x.astype(np.float64) ** 2).mean(axis=1) + 1e-6)
    np.testing.assert_allclose(rms_g, r64, rtol=2e-6, atol=0)
    assert np.all(np.abs(rms_g - rms_ref) <= np.abs(rms_ref - r64) + 2e-6 * r64)
    # Given the device's rms, every element is exact: fp32 division, fp32
    # multiply, bf16 round to nearest even.
    xh = (x / rms_g[:, None]).astype(np.float32)
    want = oracle.f32_to_bf16_bits((xh * w[None, :]).astype(np.float32))
    yb = y.view(torch.int16).cpu().numpy().view(np.uint16)
    np.testing.assert_array_equal(yb, want)
    # Against the oracle's y (sequential sum): at most one bf16 ulp apart.
    diff = np.abs(yb.astype(np.int32) - oracle.f32_to_bf16_bits(y_ref).astype(np.int32))
    assert diff.max() <= 1


def test_rmsnorm_zero_and_constant_rows_exact():
    d = 256
    x = np.zeros((2, d), np.float32)
    x[1] = np.float32(0.25)
    w = np.full(d, 2.0, np.float32)
    y, rms = norm.rms_norm_fwd(torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda())
    y_ref, _, rms_ref = oracle.rmsnorm_fwd(x, w)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(rms.cpu().numpy(), rms_ref)
    np.testing.assert_array_equal(y.view(torch.int16).cpu().numpy().view(np.uint16),
                                  oracle.f32_to_bf16_bits(y_ref))


def test_rmsnorm_70b_shape_vs_fp64_rows():
    # forward.rs:173 at the 70B layer: 8192 tokens x 8192.
    m, d = 8192, 8192
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(m, d, device="cuda", generator=g)
    w = 1.0 + 0.1 * torch.randn(d, device="cuda", generator=g)
    y, rms = norm.rms_norm_fwd(x, w)
    rows = torch.tensor([0, 1, 4095, 8191], device="cuda")
    x64 = x[rows].double()
    r64 = (x64.pow(2).mean(dim=1) + 1e-6).sqrt()
    ref = x64 / r64[:, None] * w.double()[None, :]
    torch.cuda.synchronize()
    assert torch.allclose(rms[rows].double(), r64, rtol=1e-5)
    err = (y[rows].double() - ref).abs() / ref.abs().clamp_min(1e-3)
    assert err.max().item() <= 2 ** -8


def test_rmsnorm_rejects_bad_shapes():
    x = torch.zeros(2, 6, device="cuda")
    with pytest.raises(Exception, match="d % 4"):
        norm.rms_norm_fwd(x, torch.ones(6, device="cuda"))


def test_rmsnorm_rejects_host_or_strided_outputs():
    """A caller's out / rms must be contiguous device memory: a host tensor
    or a strided view raises before any launch (the kernel would write
    through a host pointer, or over a strided rms as if contiguous)."""
    x = torch.ones(4, 8, device="cuda")
    w = torch.ones(8, device="cuda")
    good_out = torch.empty(4, 8, dtype=torch.bfloat16, device="cuda")
    good_rms = torch.empty(4, dtype=torch.float32, device="cuda")
    bad = [
        dict(out=torch.empty(4, 8, dtype=torch.bfloat16), rms=good_rms),           # host out
        dict(out=good_out, rms=torch.empty(4, dtype=torch.float32)),               # host rms
        dict(out=good_out, rms=torch.empty(8, dtype=torch.float32, device="cuda")[::2]),
        dict(out=torch.empty(8, 8, dtype=torch.bfloat16, device="cuda")[::2], rms=good_rms),
    ]
    for kw in bad:
        with pytest.raises(ValueError):
            norm.rms_norm_fwd(x, w, **kw)
    y, r = norm.rms_norm_fwd(x, w, out=good_out, rms=good_rms)
    torch.cuda.synchronize()
    assert torch.allclose(r, torch.ones_like(r), atol=1e-5)  # sqrt(1 + eps)
