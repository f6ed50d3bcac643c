"""Golden fixtures (tests/golden/fixtures.npz, written by
tests/golden/make_fixtures.py from the pinned CPU oracle on seeded BASELINE
config inputs): the oracle must reproduce them bit for bit (CPU), and the
GPU path must match them at full config size -- 64-row slices within the
parity bars and whole-output checksums (L2 norms) within 1e-4."""
import hashlib
import os
import sys

import numpy as np
import pytest

import oracle
from gpu_util import f16_to_f64, from_dev, print_case, rel_inf, to_dev

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import make_fixtures as mf  # noqa: E402

FIX = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fixtures.npz"))


def test_oracle_reproduces_the_fixtures():
    got = mf.build()
    assert set(got) == set(FIX.files)
    for k in FIX.files:
        assert np.array_equal(np.asarray(got[k]), FIX[k]), k


@pytest.mark.gpu
def test_config1_gemv_full_size(dev):
    import torch
    import jllm
    print_case("golden c1")
    W, x = mf.config1_inputs()
    Wd, xd = to_dev(W), to_dev(x)
    y = torch.empty(9728, dtype=torch.float32, device=dev)
    jllm.gemv_quant_f32(y, Wd, 12, xd, 9728, 2560)                 # MMVQ (reference gemv_quant_f32 route)
    got = from_dev(y).astype(np.float64)
    assert rel_inf(got[:64], FIX["c1_mmvq_rows0_64"]) <= 1e-3
    assert abs(np.sqrt((got ** 2).sum()) / FIX["c1_mmvq_l2"] - 1) <= 1e-4
    jllm.gemv_quant_dequant_f32(y, Wd, 12, xd, 9728, 2560)         # float dequant == gemv_quant_cpu
    got = from_dev(y).astype(np.float64)
    assert rel_inf(got[:64], FIX["c1_y_rows0_64"]) <= 1e-3
    assert abs(np.sqrt((got ** 2).sum()) / FIX["c1_y_l2"] - 1) <= 1e-4
    q = torch.zeros(2560 // 32 * 36, dtype=torch.uint8, device=dev)
    jllm.quantize_q8_1(xd, q, 2560)
    assert np.array_equal(from_dev(q), FIX["c1_q8_1"])


@pytest.mark.gpu
def test_config2_q6k_down_full_size(dev):
    import torch
    import jllm
    print_case("golden c2 down")
    W, x = mf.config2_down_inputs()
    y = torch.empty(2560, dtype=torch.float32, device=dev)
    jllm.gemv_quant_dequant_f32(y, to_dev(W), 14, to_dev(x), 2560, 9728)
    got = from_dev(y).astype(np.float64)
    assert rel_inf(got[:64], FIX["c2_down_y_rows0_64"]) <= 1e-3
    assert abs(np.sqrt((got ** 2).sum()) / FIX["c2_down_y_l2"] - 1) <= 1e-4


@pytest.mark.gpu
def test_config3_mmq_quantiser_and_product(dev):
    import torch
    import jllm
    print_case("golden c3")
    W, x = mf.config3_inputs()
    xd = to_dev(x)
    q8 = torch.zeros(2560 // 128 * 64 * 144, dtype=torch.uint8, device=dev)
    jllm.call("jllm_hip_quantize_mmq_q8_1", xd, q8, 64, 2560, 64, 1)
    h = int.from_bytes(hashlib.sha256(from_dev(q8).tobytes()).digest()[:8], "little")
    assert h == int(FIX["c3_q8_ds4_crc"])
    y = torch.empty(64 * 9728, dtype=torch.float32, device=dev)
    jllm.call("jllm_hip_gemm_quant_batched_f32", y, to_dev(W), 12, xd, 9728, 64, 2560)
    got = from_dev(y).reshape(64, 9728)[:, :64]
    assert rel_inf(got, FIX["c3_y_rows0_64"]) <= 1e-3


@pytest.mark.gpu
def test_config4_attention(dev):
    import torch
    import jllm
    print_case("golden c4")
    q, k, v, ks, vs = mf.config4_inputs()
    out = torch.empty(32 * 128, dtype=torch.int16, device=dev)
    jllm.call("jllm_hip_flash_attention_decode", out, to_dev(q), to_dev(k), to_dev(v), 32, 8, 128, 128, 512,
              1.0 / np.sqrt(128), 1, to_dev(ks), to_dev(vs), 0)
    got = f16_to_f64(from_dev(out, np.uint16))
    want = f16_to_f64(FIX["c4_out"])
    assert np.all(np.abs(got - want) <= 1e-3 * np.abs(want).max() + np.abs(want) * 2 ** -10)
