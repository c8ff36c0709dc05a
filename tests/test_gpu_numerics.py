"""Device numerics the kernels use (gfx950 hardware conversions, the library's
exp/log) against the oracle, bit for bit, on the same inputs as the host test."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from community_kv_amd import _native as nat
from oracle import numerics as nm
from tests.test_native_cpu import _floats

pytestmark = pytest.mark.gpu


def _device(op, x, out_dtype, device):
    xin = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(device)
    out = torch.empty(x.size, dtype={np.uint16: torch.int16, np.uint8: torch.uint8, np.float32: torch.float32}[out_dtype],
                      device=device)
    nat.check(nat.lib().ckv_device_numerics(op, xin.data_ptr(), out.data_ptr(), x.size,
                                            ctypes.c_void_p(nat.stream_handle(device))))
    torch.cuda.synchronize(device)
    return out.cpu().numpy().view(out_dtype)


def test_device_fp16_bf16_e4m3_match_oracle_bitwise(device):
    x = _floats()
    # f16 subnormal range and round-half-even ties around it
    x = np.concatenate([x, (np.arange(-70000, 70000, dtype=np.float32) * 2.0 ** -26)])
    assert np.array_equal(_device(2, x, np.uint16, device), nm.f32_to_f16_bits(x))
    assert np.array_equal(_device(3, x, np.uint16, device), nm.bf16_bits(x))
    assert np.array_equal(_device(4, x, np.uint8, device), nm.f32_to_e4m3(x))
    codes = np.arange(256, dtype=np.float32)
    got = _device(5, codes, np.float32, device)
    ref = nm.e4m3_to_f32(np.arange(256, dtype=np.uint8))
    finite = ~np.isnan(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.isnan(got[~finite]).all()


def test_device_exp_log_match_oracle_bitwise(device):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.uniform(-120, 0, 300_000), rng.uniform(-2, 2, 100_000), rng.uniform(0, 88, 10_000),
                        [0.0, -np.inf, np.inf, -87.3, -86.9, 88.8]]).astype(np.float32)
    assert np.array_equal(_device(0, x, np.float32, device).view(np.uint32), nm.ckv_exp(x).view(np.uint32))
    y = np.exp(rng.uniform(0, 80, 300_000)).astype(np.float32)
    y = np.concatenate([y, np.float32([1.0, 2.0, 1.41421356, 1.0000001])])
    assert np.array_equal(_device(1, y, np.float32, device).view(np.uint32), nm.ckv_log(y).view(np.uint32))
