"""ONNX TopK on the GPU against the oracle restatement.

The cases restate the reference's own TopK tests (test/ops/test_topk.py):
shapes, dtypes, axes, k values and the seeded or hand-written inputs listed
there, compared exactly (values are copies of input elements, indices are
integers).  Random cases with many ties cover the ordering rule (value, then
lower index) over every dtype, on axes up to 8192 (register and LDS
sorts) and past it (radix select, k <= 8192), and NaN inputs of either
sign.
"""
import numpy as np
import pytest
import torch

from onnxruntime_musa_amd import MoeError, topk
from oracle import oracle

pytestmark = pytest.mark.gpu


def run(cuda, x: np.ndarray, k: int, axis=-1, largest=1, torch_dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(x))
    if torch_dtype is not None:
        t = t.to(torch_dtype)
    t = t.to(cuda)
    v, i = topk(t, k, axis=axis, largest=largest)
    torch.cuda.synchronize()
    host = t.cpu()
    ref_in = host.float().numpy() if torch_dtype in (torch.float16, torch.bfloat16) else host.numpy()
    ev, ei = oracle.topk(ref_in, k, axis=axis, largest=largest)
    np.testing.assert_array_equal(i.cpu().numpy(), ei)
    gv = v.cpu()
    gv = gv.float().numpy() if torch_dtype in (torch.float16, torch.bfloat16) else gv.numpy()
    np.testing.assert_array_equal(gv, ev)
    return gv, i.cpu().numpy()


@pytest.mark.parametrize("dt", [np.float32, np.float16, np.float64, np.int32, np.int64])
def test_largest_axis_last(cuda, dt):  # test_topk.py:20-45
    x = np.array([[[1, 5, 3, 2], [4, 4, 7, 0]], [[9, 8, 8, 1], [3, 6, 2, 5]]], dtype=dt)
    run(cuda, x, 2)


def test_reference_cases(cuda):
    # :48-62 smallest along axis 1
    x = np.random.default_rng(0).standard_normal((3, 7, 5)).astype(np.float32)
    run(cuda, x, 3, axis=1, largest=0)
    # :95-126 real token-merger row, smallest, k = dim
    row = np.array([[0.0, 1.0, 9.8013570e06, 1.0715436e07, 1.0715513e07, 1.0715654e07, 1.0819043e07,
                     1.0823217e07, 0.0, 1.0, 0.0, 1.0715497e07, 1.0715646e07, 1.0849186e07]], dtype=np.float32)
    run(cuda, row, 14, largest=0)
    # :129-141 int64, dim 1024, k 512
    run(cuda, np.random.default_rng(20260710).integers(-10000, 10000, size=(2, 1024), dtype=np.int64), 512)
    # :144-155 int64 smallest with ties
    run(cuda, np.array([[5, -1, -1, 9, 0, -3, -3, 7]], dtype=np.int64), 4, largest=0)
    # :178-192 int64 dim 1300
    run(cuda, np.random.default_rng(3).integers(-2000, 2000, size=(1, 1300), dtype=np.int64), 7)
    # :195-209 integers above 2^53
    v, i = run(cuda, np.array([[2**53, 2**53 + 1, 2**53 + 2, 0]], dtype=np.int64), 2)
    np.testing.assert_array_equal(i, [[2, 1]])
    # :212-227 adjacent floats
    nxt = np.nextafter(np.float32(10.0), np.float32(np.inf))
    v, i = run(cuda, np.array([[10.0, nxt, 9.0]], dtype=np.float32), 1)
    assert i[0, 0] == 1
    # :230-246 k = 1 on a non-last axis, smallest
    v, i = run(cuda, np.array([[[4.0, 7.0], [1.0, 7.0], [1.0, 8.0], [3.0, 9.0]]], dtype=np.float32), 1, axis=1,
               largest=0)
    np.testing.assert_array_equal(i, [[[1, 0]]])
    # :249-262 double, dim 1300, two equal maxima
    x = np.random.default_rng(20260721).uniform(-4.0, 4.0, size=(2, 1300))
    x[:, 31] = 20.0
    x[:, 877] = 20.0
    run(cuda, x, 11)


@pytest.mark.parametrize("largest", [0, 1])
@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int32, np.int64])
def test_large_k(cuda, largest, dt):  # :265-289 permutation of 1300, k 1100
    x = np.random.default_rng(7).permutation(np.arange(1300)).astype(dt)[None, :]
    run(cuda, x, 1100, largest=largest)


@pytest.mark.parametrize("largest", [0, 1])
def test_ties(cuda, largest):
    run(cuda, np.full((1, 4000), 3.25, dtype=np.float32), 128, largest=largest)  # :307-323
    pattern = np.array([-3.0, -2.0, -1.0, 0.0, 1.0, 2.0, 3.0, 3.0])  # :326-340
    run(cuda, np.tile(pattern, 500).astype(np.float32)[None, :], 128, largest=largest)
    x = np.array([[5.0, 5.0, 5.0, 4.0, 4.0, 1.0, 0.0, -1.0, -1.0, -2.0, -2.0, -3.0],
                  [2.0, -4.0, 2.0, -4.0, 3.0, 3.0, 0.0, 0.0, 1.0, 1.0, -1.0, -1.0]], dtype=np.float32)
    run(cuda, x, 4, largest=largest)  # :360-395 (sorted output is a valid sorted=0 answer)
    run(cuda, np.array([[0.0, -0.0, 1.0, -0.0]], dtype=np.float32), 3, largest=largest)


@pytest.mark.parametrize("axis", [1, -2])
@pytest.mark.parametrize("k", [1, 3])
def test_axis_ties(cuda, axis, k):  # :343-357
    run(cuda, ((np.arange(40).reshape(2, 5, 4) % 7) - 3).astype(np.float32), k, axis=axis)


@pytest.mark.parametrize("shape,axis,k,dt", [
    ((1, 3999), -1, 128, np.float32), ((1, 4000), -1, 127, np.float32),
    ((1, 4000, 2), 1, 128, np.float32), ((1, 4000), -1, 128, np.float64),  # :398-421
])
def test_boundary_matrix(cuda, shape, axis, k, dt):
    run(cuda, np.random.default_rng(20260720).integers(-16, 17, size=shape).astype(dt), k, axis=axis)


@pytest.mark.parametrize("tdt", [torch.float16, torch.bfloat16])
def test_half_types(cuda, tdt):
    x = np.random.default_rng(5).integers(-50, 50, size=(64, 300)).astype(np.float32) / 8.0
    run(cuda, x, 17, torch_dtype=tdt)
    run(cuda, x, 300, largest=0, torch_dtype=tdt)


@pytest.mark.parametrize("dim", [1, 2, 63, 64, 65, 1000, 8192])
def test_dims_up_to_limit(cuda, dim):
    x = np.random.default_rng(dim).integers(-20, 20, size=(5, dim, 3)).astype(np.float32)
    run(cuda, x, min(dim, 9), axis=1)
    run(cuda, x, dim, axis=1, largest=0)


def test_many_rows_router_shape(cuda):
    x = np.random.default_rng(1).standard_normal((8192, 128)).astype(np.float32)
    run(cuda, x, 8)


def test_k_zero_and_errors(cuda):
    x = torch.ones((2, 3), device=cuda)
    v, i = topk(x, 0)
    assert v.shape == (2, 0) and i.shape == (2, 0)
    with pytest.raises(MoeError) as ei:
        topk(x, 4)
    assert ei.value.code == 2
    with pytest.raises(MoeError) as ei:
        topk(torch.ones((1, 9000), device=cuda), 8193)
    assert ei.value.code == 9


# Axes of 513..8192 with k <= 64 take the workgroup arg-max kernel (8, 16 or
# 32 entries per thread); heavy ties and -0.0 next to +0.0 exercise its order.
@pytest.mark.parametrize("largest", [0, 1])
@pytest.mark.parametrize("dim,k", [(513, 33), (600, 64), (2048, 64), (2049, 40), (4096, 64), (4097, 1),
                                   (8192, 64), (8192, 33)])
def test_workgroup_rounds(cuda, dim, k, largest):
    x = np.random.default_rng(dim + k).integers(-30, 31, size=(6, dim)).astype(np.float32)
    x[0, ::7] = -0.0
    run(cuda, x, k, largest=largest)


@pytest.mark.parametrize("dt", [np.float64, np.int32, np.int64])
def test_workgroup_rounds_dtypes(cuda, dt):
    x = np.random.default_rng(7).integers(-1000, 1000, size=(3, 3000)).astype(dt)
    run(cuda, x, 50)
    run(cuda, x.reshape(3, 1500, 2), 64, axis=1, largest=0)  # strided axis


@pytest.mark.parametrize("tdt", [torch.float16, torch.bfloat16])
def test_workgroup_rounds_half(cuda, tdt):
    x = np.random.default_rng(11).integers(-200, 200, size=(4, 5000)).astype(np.float32) / 16.0
    run(cuda, x, 48, torch_dtype=tdt)


def test_workgroup_rounds_many_slices(cuda):
    x = np.random.default_rng(12).standard_normal((700, 1024)).astype(np.float32)
    run(cuda, x, 64)


# Many slices through the wave kernel, at lane groups of 4, 16, 4 and 32.
@pytest.mark.parametrize("rows,dim,k", [(70000, 20, 2), (32768, 100, 5), (20000, 30, 3), (5000, 250, 32)])
def test_wave_entries_per_lane(cuda, rows, dim, k):
    x = np.random.default_rng(rows).integers(-40, 41, size=(rows, dim)).astype(np.float32)
    run(cuda, x, k)


# Axes longer than 8192 take the radix select (k <= 8192).
def test_large_last_axis_k192(cuda):  # test_topk.py:65-77, the seeded 1 x 20000 case
    x = np.random.default_rng(20260703).uniform(-1.0, 1.0, size=(1, 20000)).astype(np.float32)
    run(cuda, x, 192)


@pytest.mark.parametrize("largest", [0, 1])
@pytest.mark.parametrize("rows,dim,k", [(3, 8193, 1), (2, 20000, 8192), (5, 50000, 700), (4, 100003, 33),
                                        (1, 300000, 2048)])
def test_radix_select(cuda, rows, dim, k, largest):
    # integer-valued floats: long runs of ties at the k-th key, taken in index order
    x = np.random.default_rng(dim + k).integers(-3000, 3000, size=(rows, dim)).astype(np.float32)
    x[0, ::5] = -0.0
    run(cuda, x, k, largest=largest)


@pytest.mark.parametrize("dt", [np.float64, np.int32, np.int64])
def test_radix_select_dtypes(cuda, dt):
    x = np.random.default_rng(5).integers(-100000, 100000, size=(3, 12000)).astype(dt)
    run(cuda, x, 300)
    run(cuda, x.reshape(3, 4, 3000).transpose(0, 2, 1).copy().reshape(3, 3000, 4), 9, axis=1, largest=0)
    big = np.random.default_rng(6).integers(-2**62, 2**62, size=(2, 9000), dtype=np.int64)
    if dt == np.int64:
        run(cuda, big, 100)


@pytest.mark.parametrize("tdt", [torch.float16, torch.bfloat16])
def test_radix_select_half(cuda, tdt):
    x = np.random.default_rng(13).integers(-500, 500, size=(2, 30000)).astype(np.float32) / 8.0
    run(cuda, x, 1000, torch_dtype=tdt)
    run(cuda, x, 500, largest=0, torch_dtype=tdt)


def test_all_equal_long_axis(cuda):  # the all-equal rule of test_topk.py:307-323 past 8192
    run(cuda, np.full((2, 40000), 3.25, dtype=np.float32), 128)
    run(cuda, np.full((2, 40000), 3.25, dtype=np.float32), 128, largest=0)


# NaN of either sign (and any payload) has one key above +inf: NaNs come
# first for largest = 1 and last for largest = 0, among themselves in index
# order.  The reference's comparator leaves NaN unordered, so this is the
# library's rule, checked against an explicit construction.
def _nan_expected(x: np.ndarray, k: int, largest: int):
    out_v, out_i = [], []
    for row in x:
        nan = [i for i in range(row.size) if np.isnan(row[i])]
        num = [i for i in range(row.size) if not np.isnan(row[i])]
        key = (lambda i: (-(float(row[i]) + 0.0), i)) if largest else (lambda i: (float(row[i]) + 0.0, i))
        order = (nan + sorted(num, key=key)) if largest else (sorted(num, key=key) + nan)
        out_i.append(order[:k])
        out_v.append(row[order[:k]])
    return np.array(out_v), np.array(out_i, dtype=np.int64)


@pytest.mark.parametrize("largest", [0, 1])
@pytest.mark.parametrize("dim,k", [(100, 10), (3000, 40), (3000, 200), (20000, 300)])  # wave, workgroup, bitonic, radix
def test_nan_order(cuda, dim, k, largest):
    rng = np.random.default_rng(dim + k)
    x = rng.standard_normal((3, dim)).astype(np.float32)
    for r in range(3):
        pos = rng.choice(dim, size=7, replace=False)
        x[r, pos[:4]] = np.nan
        x[r, pos[4:]] = -np.nan
    x[1, :3] = np.array([0x7FC00001, 0xFFC12345, 0x7FFFFFFF], np.uint32).view(np.float32)  # payloads
    x[2, 5] = np.inf
    t = torch.from_numpy(x).to(cuda)
    v, i = topk(t, k, largest=largest)
    torch.cuda.synchronize()
    ev, ei = _nan_expected(x, k, largest)
    np.testing.assert_array_equal(i.cpu().numpy(), ei)
    np.testing.assert_array_equal(v.cpu().numpy().view(np.uint32), ev.view(np.uint32))  # exact bits kept
