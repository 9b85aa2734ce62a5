"""ONNX Softmax on the GPU against the float64 oracle.

The cases restate the reference's Softmax tests (test/ops/test_softmax.py):
shapes, axes, dtypes and seeds, with its tolerances (fp32 1e-5 relative /
1e-6 absolute as the CPU-vs-device default of op_test_utils, fp16 and bf16
2e-2, double 1e-6 / 1e-7), plus long rows, strided axes and the router's
shape.
"""
import numpy as np
import pytest
import torch

from onnxruntime_musa_amd import softmax
from oracle import oracle

pytestmark = pytest.mark.gpu

TOL = {torch.float32: (1e-5, 1e-6), torch.float16: (2e-2, 2e-2), torch.bfloat16: (2e-2, 2e-2),
       torch.float64: (1e-6, 1e-7)}


def run(cuda, x: np.ndarray, axis=-1, dt=torch.float32):
    t = torch.from_numpy(np.ascontiguousarray(x)).to(dt).to(cuda)
    y = softmax(t, axis)
    torch.cuda.synchronize()
    ref = oracle.softmax(t.cpu().double().numpy(), axis)
    rtol, atol = TOL[dt]
    np.testing.assert_allclose(y.cpu().double().numpy(), ref, rtol=rtol, atol=atol)


def test_reference_cases(cuda):
    run(cuda, np.random.default_rng(0).standard_normal((16, 32)), -1)      # :14-22
    run(cuda, np.random.default_rng(1).standard_normal((16, 32)), 0)       # :25-33
    run(cuda, np.random.default_rng(2).standard_normal((2, 5, 4)), 1)      # :36-44
    run(cuda, np.random.default_rng(3).standard_normal((32,)))             # :47-49
    run(cuda, np.random.default_rng(4).standard_normal((8, 16)), -1, torch.float16)   # :52-62
    run(cuda, np.random.default_rng(5).standard_normal((8, 16)), -1, torch.float64)   # :65-75
    run(cuda, np.random.default_rng(6).standard_normal((4, 8)), -1, torch.bfloat16)   # :78-112


@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16, torch.float64])
@pytest.mark.parametrize("shape,axis", [((3, 1000), -1), ((7, 4097), 1), ((5, 6, 33), 1), ((2, 300, 4), 0),
                                        ((8192, 128), -1), ((1, 1), 0),
                                        ((3, 256), -1), ((4, 257), -1), ((3, 1500), -1), ((4, 2048), -1), ((9, 2500), -1), ((5, 4096), -1),
                                        ((7, 6000), -1), ((3, 8192), -1), ((5, 8193), -1), ((2, 16384), -1),
                                        ((3, 16385), -1), ((2, 33000), -1)])
def test_shapes(cuda, dt, shape, axis):
    run(cuda, 3.0 * np.random.default_rng(sum(shape)).standard_normal(shape), axis, dt)


def test_large_values_are_shift_invariant(cuda):
    x = np.random.default_rng(9).standard_normal((4, 64)) + 80.0
    run(cuda, x, -1)


@pytest.mark.parametrize("dim", [200, 3000, 5000, 12000, 20000])
def test_masked_rows(cuda, dim):
    # -inf (masked) entries, some rows led by a masked prefix, one row all but one masked
    x = np.random.default_rng(dim).standard_normal((6, dim)).astype(np.float32)
    x[0, : dim // 2] = -np.inf
    x[1, ::3] = -np.inf
    x[2, :-1] = -np.inf
    t = torch.from_numpy(x).to(cuda)
    y = softmax(t, -1)
    torch.cuda.synchronize()
    ref = oracle.softmax(x.astype(np.float64), -1)
    got = y.cpu().double().numpy()
    assert np.all(np.isfinite(got))
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)


def test_masked_strided_axis(cuda):
    # a middle axis (one thread per (outer, inner) position) with masked prefixes
    x = np.random.default_rng(77).standard_normal((4, 500, 3)).astype(np.float32)
    x[0, :250, :] = -np.inf
    x[1, ::3, 1] = -np.inf
    x[2, :-1, 2] = -np.inf
    t = torch.from_numpy(x).to(cuda)
    y = softmax(t, 1)
    torch.cuda.synchronize()
    got = y.cpu().double().numpy()
    assert np.all(np.isfinite(got))
    np.testing.assert_allclose(got, oracle.softmax(x.astype(np.float64), 1), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dt", [torch.float32, torch.float64])
def test_long_strided_axis(cuda, dt):
    run(cuda, 4.0 * np.random.default_rng(78).standard_normal((16, 3000, 40)), 1, dt)
