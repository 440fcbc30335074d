"""GPU parity of on-device re-quantization (weights changed by an update step,
doublepass/src/precision.rs:187-202, before their write-back,
flowcast/src/lib.rs:501-521): the bf16-input quantize and the fused
quantize + double-quant are bit-exact against the oracle's quantize
(quantizer.py:21-53) and double-quant encode, and requantize_ writes into the
weight's own buffers."""
import numpy as np
import pytest
import torch

import oracle
from aethelstream_amd import nf4

pytestmark = pytest.mark.gpu
DEV = "cuda"

SIZES = [1, 63, 64, 65, 1001, 64 * 256, 64 * 256 * 3 + 64 * 5 + 17]


def _values(n, seed, bf16):
    x = oracle.gen_normal(seed, n, 0.02)
    if n >= 64 * 3:
        x[64:128] = 0.0                    # an all-zero block
        x[128:192] *= 1e-9                 # absmax below the 1e-8 clamp
    t = torch.from_numpy(x).to(DEV)
    if bf16:
        t = t.to(torch.bfloat16)
    # What the oracle quantizes: the same values in fp32 (bf16 widens exactly).
    return t, t.float().cpu().numpy()


def _u32(t):
    return t.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("n", SIZES)
def test_quantize_bf16_input_vs_oracle(n):
    t, ref_in = _values(n, 100 + n, bf16=True)
    r = nf4.quantize_nf4(t)
    pk_ref, am_ref = oracle.quantize_nf4(ref_in)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(r.packed.cpu().numpy(), pk_ref)
    np.testing.assert_array_equal(_u32(r.absmax), am_ref.view(np.uint32))


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("group", [1, 4, 256, 8192])
@pytest.mark.parametrize("bf16", [False, True])
def test_quantize_dq_fused_vs_oracle(n, group, bf16):
    t, ref_in = _values(n, 200 + n + group, bf16)
    w = nf4.quantize_weight(t, double_quant=True, dq_group=group)
    pk_ref, am_ref = oracle.quantize_nf4(ref_in)
    q_ref, s_ref = oracle.dq_encode(am_ref, group)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(w.packed.cpu().numpy(), pk_ref)
    np.testing.assert_array_equal(w.absmax_q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(_u32(w.absmax_scale), s_ref.view(np.uint32))



@pytest.mark.parametrize("group,bf16", [(8, False), (16, True), (256, False)])
def test_quantize_dq_more_groups_than_workgroups(group, bf16):
    # The fused kernel's workgroups each take several groups in turn once
    # there are more groups than its grid (at most 1024 workgroups): 3001+
    # groups, a partial last group and a partial last block.
    n = 64 * group * 3001 + 64 * 3 + 17 if group < 256 else 64 * 256 * 1100 + 100
    print(f"quantize_dq many groups group={group} bf16={bf16} n={n}", flush=True)
    t, ref_in = _values(n, 900 + group, bf16)
    w = nf4.quantize_weight(t, double_quant=True, dq_group=group)
    pk_ref, am_ref = oracle.quantize_nf4(ref_in)
    q_ref, s_ref = oracle.dq_encode(am_ref, group)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(w.packed.cpu().numpy(), pk_ref)
    np.testing.assert_array_equal(w.absmax_q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(_u32(w.absmax_scale), s_ref.view(np.uint32))

def test_fused_equals_two_launch_path():
    # The fused kernel and quantize_nf4 + dq_encode on the same device values.
    t, _ = _values(64 * 1000 + 3, 7, bf16=False)
    w = nf4.quantize_weight(t, double_quant=True, dq_group=256)
    r = nf4.quantize_nf4(t)
    q, s = nf4.dq_encode(r.absmax, 256)
    torch.cuda.synchronize()
    assert torch.equal(w.packed, r.packed)
    assert torch.equal(w.absmax_q, q)
    assert torch.equal(w.absmax_scale.view(torch.int32), s.view(torch.int32))


@pytest.mark.parametrize("dq", [False, True])
@pytest.mark.parametrize("bf16", [False, True])
def test_requantize_in_place(dq, bf16):
    n, k = 384, 512
    a, _ = _values(n * k, 11, bf16)
    b, b_ref = _values(n * k, 12, bf16)
    w = nf4.quantize_weight(a.view(n, k), double_quant=dq)
    ptrs = [w.packed.data_ptr()] + ([w.absmax_q.data_ptr(), w.absmax_scale.data_ptr()] if dq
                                    else [w.absmax.data_ptr()])
    nf4.requantize_(w, b.view(n, k))
    fresh = nf4.quantize_weight(b.view(n, k), double_quant=dq)
    torch.cuda.synchronize()
    assert ptrs == [w.packed.data_ptr()] + ([w.absmax_q.data_ptr(), w.absmax_scale.data_ptr()]
                                            if dq else [w.absmax.data_ptr()])
    assert torch.equal(w.packed, fresh.packed)
    if dq:
        assert torch.equal(w.absmax_q, fresh.absmax_q)
        assert torch.equal(w.absmax_scale.view(torch.int32), fresh.absmax_scale.view(torch.int32))
    else:
        np.testing.assert_array_equal(_u32(w.absmax), oracle.quantize_nf4(b_ref)[1].view(np.uint32))
    # The re-quantized weight dequantizes like the oracle's.
    pk_ref, am_ref = oracle.quantize_nf4(b_ref)
    if dq:
        am_ref = oracle.dq_decode(*oracle.dq_encode(am_ref, w.dq_group), w.dq_group)
    got = nf4.dequant(w).view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
    np.testing.assert_array_equal(got, oracle.dequant_bf16(pk_ref, am_ref, n * k))


def test_requantize_argument_errors():
    w = nf4.quantize_weight(torch.zeros(64, 64, device=DEV), double_quant=True)
    with pytest.raises(ValueError):
        nf4.requantize_(w, torch.zeros(64 * 63, device=DEV))
    with pytest.raises(ValueError):
        nf4.requantize_(w, torch.zeros(64 * 64, device=DEV, dtype=torch.float16))
