"""Pins the oracle's residual-block pieces (oracle.layernorm / silu /
round_to) against torch's CPU layer_norm and silu (library routines) and
closed forms, before they check the GPU block."""
import numpy as np
import pytest


def test_layernorm_matches_torch_and_closed_forms():
    import oracle
    import torch

    rng = np.random.default_rng(0)
    x = (rng.standard_normal((64, 128)) * 3 + 1).astype(np.float32)
    g = rng.standard_normal(128).astype(np.float32)
    b = rng.standard_normal(128).astype(np.float32)
    ref = torch.nn.functional.layer_norm(torch.from_numpy(x), (128,), torch.from_numpy(g),
                                         torch.from_numpy(b), eps=1e-6).numpy()
    assert np.allclose(oracle.layernorm(x, g, b, 1e-6), ref, rtol=1e-5, atol=1e-5)
    y = oracle.layernorm(x)
    assert np.allclose(y.mean(axis=1), 0, atol=1e-5)
    assert np.allclose(y.var(axis=1), 1, atol=1e-3)
    assert np.array_equal(oracle.layernorm(np.full((2, 8), 5.0, np.float32)), np.zeros((2, 8), np.float32))


def test_silu_matches_torch_and_closed_forms():
    import oracle
    import torch

    x = np.linspace(-20, 20, 4001, dtype=np.float32)
    assert np.allclose(oracle.silu(x), torch.nn.functional.silu(torch.from_numpy(x)).numpy(),
                       rtol=1e-6, atol=1e-7)
    assert oracle.silu(np.zeros(1, np.float32))[0] == 0.0
    assert abs(oracle.silu(np.float32([30.0]))[0] - 30.0) < 1e-5


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_round_to_matches_torch_casts(orc, dt):
    import oracle
    import torch

    x = np.random.default_rng(1).standard_normal(10000).astype(np.float32) * 100
    code = {"bf16": oracle.BF16, "f16": oracle.F16, "f32": oracle.F32}[dt]
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dt]
    want = torch.from_numpy(x).to(tdt).float().numpy()
    assert np.array_equal(oracle.round_to(orc, x, code), want)
