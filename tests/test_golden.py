"""The committed golden fixtures agree with the oracle and with nested eager autograd."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from golden_cases import CASE_NAMES, load_case
from oracle import jet, torch_ref


@pytest.mark.parametrize("name", CASE_NAMES)
def test_fixture_reproduces_with_oracle(name: str) -> None:
    case = load_case(name)
    flat = case["parameters"].astype(np.float64)
    x = case["coordinates"].astype(np.float64)
    u, lap = jet.forward(flat, x)
    np.testing.assert_array_equal(u, case["u"])
    np.testing.assert_array_equal(lap, case["laplacian"])
    gp, gx = jet.backward(flat, x, case["grad_output"], case["grad_laplacian"])
    np.testing.assert_allclose(gp, case["grad_parameters"], rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(gx, case["grad_coordinates"], rtol=1e-13, atol=1e-15)


@pytest.mark.parametrize("name", CASE_NAMES)
def test_fixture_matches_nested_autograd(name: str) -> None:
    case = load_case(name)
    flat = torch.tensor(case["parameters"].astype(np.float64), requires_grad=True)
    x = torch.tensor(case["coordinates"].astype(np.float64))
    u, lap = torch_ref.eager_laplacian(flat, x, create_graph=True)
    np.testing.assert_allclose(u.detach().numpy().ravel(), case["u"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lap.detach().numpy().ravel(), case["laplacian"], rtol=1e-10, atol=1e-10)
    gu = torch.tensor(case["grad_output"].astype(np.float64))
    gl = torch.tensor(case["grad_laplacian"].astype(np.float64))
    loss = (gu * u.ravel()).sum() + (gl * lap.ravel()).sum()
    (gp,) = torch.autograd.grad(loss, flat)
    expected = case["grad_parameters"]
    np.testing.assert_allclose(gp.numpy(), expected, rtol=1e-9, atol=1e-11 * np.abs(expected).max())
