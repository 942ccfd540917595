"""GPU parity against the committed golden vectors (tests/golden/*.npz): each fixture's inputs
through the HIP path, its stored oracle output and float64 closed form as the expected values.
Tolerances (max-abs): 1e-4 for f32 operands (f16 K/V widened to f32 included), 2e-2 for bf16.
"""

from __future__ import annotations

import glob
import os

import numpy as np
import pytest
import torch

from ffai_amd import flash_attn as fa
from tests.helpers import TOL_BF16, TOL_F32, max_abs

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _bf16_dev(bits: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits.astype(np.int16))).to(device).view(torch.bfloat16)


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "*.npz"))),
                         ids=lambda p: os.path.basename(p))
def test_golden_vector_on_gpu(gpu, path):
    z = np.load(path, allow_pickle=False)
    name = os.path.basename(path)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    if name.startswith("encoder_f32"):
        q = dev(z["q"])
        got = fa.attend_merged(q, dev(z["kt"]), dev(z["v"]))  # (1, T, H*64), merged
        assert got is not None
        h, t = q.shape[1], q.shape[2]
        got = got.reshape(1, t, h, 64).permute(0, 2, 1, 3).cpu().numpy()
        tol = TOL_F32
    elif name.startswith("decode_f32"):
        got = fa.attend(dev(z["q"]), dev(z["kt"]), dev(z["v"]))
        assert got is not None
        got = got.cpu().numpy()
        tol = TOL_F32
    elif name.startswith("decode_f16kv"):
        got = fa.attend(dev(z["q"]), dev(z["kt16"]), dev(z["v16"]))
        assert got is not None
        got = got.cpu().numpy()
        tol = TOL_F32
    elif name.startswith("causal_gqa"):
        got = fa.attention(_bf16_dev(z["q_bf16"], gpu), _bf16_dev(z["k_bf16"], gpu),
                           _bf16_dev(z["v_bf16"], gpu), scale=float(z["scale"]), causal=True,
                           out_dtype=torch.float32).cpu().numpy()
        tol = TOL_BF16
    elif name.startswith("ragged_beams"):
        lens = torch.from_numpy(z["lens"]).to(gpu)
        got = fa.attention(_bf16_dev(z["q_bf16"], gpu), _bf16_dev(z["k_bf16"], gpu),
                           _bf16_dev(z["v_bf16"], gpu), scale=float(z["scale"]), kv_lens=lens,
                           out_dtype=torch.float32).cpu().numpy()
        tol = TOL_BF16
    elif name.startswith("encoder_bf16"):
        full = fa.attention(_bf16_dev(z["q_bf16"], gpu), _bf16_dev(z["kt_bf16"], gpu),
                            _bf16_dev(z["v_bf16"], gpu), k_transposed=True,
                            scale=float(z["scale"]), out_dtype=torch.float32)
        got = full[:, :, torch.from_numpy(z["rows"]).long().to(gpu)].cpu().numpy()
        tol = TOL_BF16
    else:
        pytest.fail(f"unknown fixture {name}")
    err_oracle, err_f64 = max_abs(got, z["out"]), max_abs(got, z["f64"])
    print(f"{name}: {err_oracle:.3e} against the oracle, {err_f64:.3e} against the closed form")
    assert err_oracle < tol and err_f64 < tol
