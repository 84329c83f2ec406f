"""GPU parity of the Timestral variate attention (tsfm_variate_attend) against the oracle's
restatement of VariateJob.run (src/timestral/model.zig:648-709) and nn.mulSigmoid
(src/core/nn.zig:423-433), through the C ABI.

Bar: scaled error max|gpu - oracle| / max(|oracle|, 1) <= 1e-5 (the f32 tolerance). Covered: row
counts 1..16 that one 16-slot score block takes (several heads per block below 16 rows, a partial
last head block), and 17, 24, 33 and the largest count, 256, where 16-row query blocks walk 16-row
key blocks with an online softmax; with and without the covariate firewalls, encoder and decoder
slots, the fused sigmoid gate, host and device pointers, and the singleton case o = v exactly.
"""
import numpy as np
import pytest

import _ref

pytestmark = pytest.mark.gpu

TOL = 1e-5
THREADS = 16


def _inputs(seed, groups, vall, ne, h, d, p_valid=0.7):
    rng = np.random.default_rng(seed)
    sl = ne + h
    qkv = rng.standard_normal((groups * vall, sl, 3 * d)).astype(np.float32)
    kv = (rng.random((groups * vall, ne)) < p_valid).astype(np.uint8)
    return qkv, kv


def _roles(vall):
    return np.array(([_ref.ROLE_TARGET, _ref.ROLE_PAST, _ref.ROLE_KNOWN, _ref.ROLE_PAST] * 64)[:vall], np.uint8)


def _oracle(orc, qkv, kv, roles, cov, groups, vall, ne, h, d, nh, gate=None):
    want = np.zeros((groups * vall, ne + h, d), np.float32)
    orc.timestral_variate_attention(THREADS, qkv, want, kv, roles, cov, groups, vall, ne, h, d, nh, 64)
    if gate is not None:
        orc.mul_sigmoid(want, want, gate)
    return want


@pytest.mark.parametrize("cov", [False, True])
@pytest.mark.parametrize("vall", [1, 2, 3, 4, 5, 8, 13, 16, 17, 24, 33])
def test_variate_matches_oracle(ta, orc, gpu_ready, vall, cov):
    groups, ne, h, nh = 3, 21, 5, 4
    d = nh * 64
    qkv, kv = _inputs(vall + 17 * cov, groups, vall, ne, h, d)
    roles = _roles(vall)
    o = np.full((groups * vall, ne + h, d), -7.0, np.float32)
    rc = ta.timestral_variate_attention(qkv, o, kv, roles, cov, groups, vall, ne, h, d, nh, 64)
    assert rc == ta.OK, ta.last_error()
    want = _oracle(orc, qkv, kv, roles, cov, groups, vall, ne, h, d, nh)
    assert _ref.scaled_err(o, want) <= TOL


@pytest.mark.parametrize("vall,nh", [(4, 5), (3, 7), (16, 3)])
def test_variate_partial_head_block(ta, orc, gpu_ready, vall, nh):
    """Head counts that do not fill the last block of 16 // vall heads."""
    groups, ne, h = 2, 9, 3
    d = nh * 64
    qkv, kv = _inputs(31 + vall, groups, vall, ne, h, d)
    roles = _roles(vall)
    o = np.zeros((groups * vall, ne + h, d), np.float32)
    assert ta.timestral_variate_attention(qkv, o, kv, roles, True, groups, vall, ne, h, d, nh, 64) == ta.OK
    assert _ref.scaled_err(o, _oracle(orc, qkv, kv, roles, True, groups, vall, ne, h, d, nh)) <= TOL


@pytest.mark.parametrize("vall,nh,cov", [(24, 3, True), (256, 2, True), (40, 2, False)])
def test_variate_many_rows_gate_and_device_pointers(ta, orc, gpu_ready, vall, nh, cov):
    """More than 16 rows per series: the row-block kernel, with the gate, on device tensors and
    host arrays (the same bits), against the oracle."""
    import torch

    groups, ne, h = 2, 11, 3
    d = nh * 64
    qkv, kv = _inputs(70 + vall, groups, vall, ne, h, d, p_valid=0.4)
    gate = (np.random.default_rng(71).standard_normal((groups * vall, ne + h, d)) * 3).astype(np.float32)
    roles = _roles(vall)
    want = _oracle(orc, qkv, kv, roles, cov, groups, vall, ne, h, d, nh, gate)
    o = np.zeros_like(want)
    assert ta.timestral_variate_attention(qkv, o, kv, roles, cov, groups, vall, ne, h, d, nh, 64, gate=gate) == ta.OK
    assert _ref.scaled_err(o, want) <= TOL
    dev = {n: torch.from_numpy(x).cuda() for n, x in dict(qkv=qkv, kv=kv, gate=gate).items()}
    od = torch.zeros(want.shape, dtype=torch.float32, device="cuda")
    assert ta.timestral_variate_attention(dev["qkv"], od, dev["kv"], roles, cov, groups, vall, ne, h, d, nh, 64,
                                          gate=dev["gate"]) == ta.OK
    torch.cuda.synchronize()
    assert np.array_equal(od.cpu().numpy(), o)


def test_variate_gate_and_device_pointers(ta, orc, gpu_ready):
    """The fused gate (o * sigmoid(gate)), with device tensors, equals the host-pointer call."""
    import torch

    groups, vall, ne, h, nh = 4, 4, 33, 7, 16
    d = nh * 64
    qkv, kv = _inputs(44, groups, vall, ne, h, d)
    gate = (np.random.default_rng(45).standard_normal((groups * vall, ne + h, d)) * 3).astype(np.float32)
    roles = _roles(vall)
    want = _oracle(orc, qkv, kv, roles, True, groups, vall, ne, h, d, nh, gate)
    o = np.zeros_like(want)
    assert ta.timestral_variate_attention(qkv, o, kv, roles, True, groups, vall, ne, h, d, nh, 64, gate=gate) == ta.OK
    assert _ref.scaled_err(o, want) <= TOL
    dev = {n: torch.from_numpy(x).cuda() for n, x in dict(qkv=qkv, kv=kv, gate=gate).items()}
    od = torch.zeros(want.shape, dtype=torch.float32, device="cuda")
    rc = ta.timestral_variate_attention(dev["qkv"], od, dev["kv"], roles, True, groups, vall, ne, h, d, nh, 64,
                                        gate=dev["gate"])
    assert rc == ta.OK, ta.last_error()
    torch.cuda.synchronize()
    assert np.array_equal(od.cpu().numpy(), o)


def test_variate_singleton_is_exactly_v(ta, gpu_ready):
    groups, ne, h, nh = 5, 12, 4, 2
    d = nh * 64
    qkv, kv = _inputs(50, groups, 1, ne, h, d, p_valid=0.0)
    o = np.zeros((groups, ne + h, d), np.float32)
    assert ta.timestral_variate_attention(qkv, o, kv, [0], False, groups, 1, ne, h, d, nh, 64) == ta.OK
    assert np.array_equal(o, qkv[:, :, 2 * d:])


def test_variate_rows_past_the_largest_count_are_refused(ta, gpu_ready):
    groups, vall, ne, h, nh = 1, ta.VARIATE_MAX_ROWS + 1, 4, 0, 1
    d = nh * 64
    qkv, kv = _inputs(51, groups, vall, ne, h, d)
    o = np.zeros((vall, ne + h, d), np.float32)
    assert ta.timestral_variate_attention(qkv, o, kv, [0] * vall, False, groups, vall, ne, h, d, nh, 64) == ta.E_UNSUPPORTED
