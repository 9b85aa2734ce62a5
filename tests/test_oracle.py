"""Pins the CPU oracle (oracle/moe_oracle.c) before it is trusted as the checker.

Each oracle function is checked against something that does not restate it:

  conversions  numpy's IEEE fp16 (exhaustive for fp16 -> fp32), known bf16 RNE
               values, the reference's bf16 helper formula
               (test/ops/op_test_utils.py:235-245)
  orc_route    the reference's TopK known-answer vectors
               (test/ops/test_topk.py:212-227, 230-246, 307-323), float64
               closed-form softmax / sigmoid, k = E full order, normalised
               k = 1 weight 1
  orc_dispatch brute force (a stable sort by expert) on every routing of tiny
               shapes, invariants on large random routings
  orc_dequant  hand-packed bytes (0x80 -> 0 for int8; 0x78 -> 0, -1 for int4),
               block-boundary scale indexing, and a round trip through the
               symmetric encoder written independently in float64 numpy
               (every weight back within half a step, each row's / block's
               peak exactly +-127 s / +-7 s, for int8/int4 x per-channel /
               block 16/32/128 x f16/bf16/f32 scales)
  activations  closed forms at fixed points (SiLU, erf-GELU); SwiGLU reduces
               to textbook Swish-GLU at alpha 1, beta 0, no limit, and to
               relu gating as alpha grows; clamp saturation of both inputs
  forward      an independent float64 numpy formulation (dense matmuls),
               layout equivalences (fc1/fc3 unfused == fused chunked ==
               fused interleaved), QMoE == MoE on dequantised weights,
               single-expert == dense FFN, linearity in the fc2 scales
  mxfp4        E2M1 / E8M0 known answers (all 16 codes, scale bytes 0, 126,
               127, 128, 254, 255 = NaN), hand-packed bytes, a round trip
               through the MX v1.0 quantizer written here in numpy (nearest
               value within half a grid step, saturation past 6) with planted
               nibble-order, sign and scale-bias mistakes, and the forward
               against a float64 formulation decoding with numpy's own table
  fixtures     tests/golden/*.npz written by tests/golden/make_golden.py

The "planted mistake" tests feed each check a plausible mistake (swapped tie
order, unstable dispatch, high-nibble-first decode, a zero point off by one,
block scales along the wrong axis, dropped bias, swapped gate/linear halves)
on the CPU and assert that the check rejects it.
"""
import itertools
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---------------------------------------------------------------- conversions
def test_f16_to_f32_exhaustive():
    lib = oracle.load()
    bits = np.arange(65536, dtype=np.uint32)
    got = np.array([lib.orc_f16_to_f32(int(b)) for b in bits], np.float32)
    exp = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(exp)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), exp[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy_rne():
    lib = oracle.load()
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(100),
        rng.standard_normal(5000).astype(np.float32) * np.float32(1e-5),   # fp16 subnormal range
        np.array([65504, 65519.99, 65520, 65536, 1e-8, 5.96e-8, 2.98e-8, 2.99e-8, -0.0, np.inf, -np.inf],
                 np.float32),
        # exact halfway points between fp16 neighbours
        (np.arange(1024, 1100, dtype=np.float32) + np.float32(0.5)),
    ])
    got = np.array([lib.orc_f32_to_f16(float(v)) for v in vals], np.uint16)
    exp = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("f,bits", [(1.0, 0x3F80), (-2.0, 0xC000), (1.00390625, 0x3F80),
                                    (1.01171875, 0x3F82), (3.0e38, 0x7F62)])
def test_bf16_known_values(f, bits):
    assert oracle.load().orc_f32_to_bf16(f) == bits
    back = np.array([bits << 16], np.uint32).view(np.float32)[0]
    assert np.float32(oracle.load().orc_bf16_to_f32(bits)) == back


def test_bf16_matches_reference_helper():
    lib = oracle.load()
    rng = np.random.default_rng(1)
    vals = rng.standard_normal(5000).astype(np.float32) * np.float32(7)
    got = np.array([lib.orc_f32_to_bf16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, oracle.f32_to_bf16_bits(vals))


# ---------------------------------------------------------------- router
def test_topk_kat_ties_go_to_lower_index():
    # test_topk.py:230-246 (k=1 along an axis with equal maxima)
    ids, _ = oracle.route(np.array([[4.0, 7.0, 1.0, 7.0], [9.0, 1.0, 9.0, 8.0]]), 1)
    assert ids[:, 0].tolist() == [1, 0]


@pytest.mark.parametrize("E,k", [(8, 2), (4000, 128)])
def test_topk_kat_all_equal_gives_arange(E, k):
    # test_topk.py:307-323
    ids, _ = oracle.route(np.full((2, E), 3.25, np.float32), k)
    assert np.array_equal(ids, np.tile(np.arange(k), (2, 1)))


def test_topk_kat_adjacent_floats_are_not_ties():
    # test_topk.py:212-227
    nxt = np.nextafter(np.float32(10.0), np.float32(np.inf))
    ids, _ = oracle.route(np.array([[10.0, nxt, 9.0]], np.float32), 1)
    assert ids.tolist() == [[1]]


def test_route_k_equals_e_is_stable_argsort():
    rng = np.random.default_rng(2)
    lg = np.round(rng.standard_normal((50, 9)) * 2).astype(np.float32)  # many ties
    ids, _ = oracle.route(lg, 9)
    assert np.array_equal(ids, np.argsort(-lg, axis=1, kind="stable"))


@pytest.mark.parametrize("normalize", [0, 1])
def test_route_softmax_closed_form(normalize):
    rng = np.random.default_rng(3)
    lg = rng.standard_normal((200, 16)).astype(np.float32)
    ids, w = oracle.route(lg, 4, normalize=bool(normalize))
    l64 = lg.astype(np.float64)
    p = np.exp(l64 - l64.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    sel = np.take_along_axis(p, ids, 1)
    if normalize:
        sel /= sel.sum(1, keepdims=True)
    np.testing.assert_allclose(w, sel, rtol=1e-6)


def test_route_sigmoid_closed_form():
    rng = np.random.default_rng(4)
    lg = rng.standard_normal((100, 8)).astype(np.float32)
    ids, w = oracle.route(lg, 3, sigmoid=True)
    np.testing.assert_allclose(w, 1 / (1 + np.exp(-np.take_along_axis(lg.astype(np.float64), ids, 1))), rtol=1e-6)


def test_route_normalized_k1_weight_is_one():
    rng = np.random.default_rng(5)
    _, w = oracle.route(rng.standard_normal((40, 8)).astype(np.float32), 1, normalize=True)
    assert np.all(w == 1.0)


def test_route_nan_ranks_last():
    lg = np.array([[np.nan, 1.0, -5.0, np.nan]], np.float32)
    ids, _ = oracle.route(lg, 4)
    assert ids.tolist() == [[1, 2, 0, 3]]


def test_planted_tie_mistake_is_caught():
    """A router that breaks ties toward the higher id fails the KAT."""
    lg = np.array([[4.0, 7.0, 1.0, 7.0]], np.float32)
    mutant = np.argsort(-lg[:, ::-1], axis=1, kind="stable")[:, :1]
    mutant = lg.shape[1] - 1 - mutant
    ids, _ = oracle.route(lg, 1)
    assert mutant.tolist() == [[3]] and ids.tolist() == [[1]]


# ---------------------------------------------------------------- dispatch
def _brute_dispatch(ids, E):
    flat = ids.reshape(-1)
    perm = sorted(range(flat.size), key=lambda f: (flat[f], f))
    offs = [0] + list(np.cumsum(np.bincount(flat, minlength=E)))
    return np.array(offs, np.int32), np.array(perm, np.int32)


def test_dispatch_brute_force_all_tiny_routings():
    n = 0
    for E, k, T in [(1, 1, 3), (2, 1, 3), (3, 2, 3), (4, 2, 3), (3, 3, 2)]:
        choices = [c for c in itertools.permutations(range(E), k)]
        for combo in itertools.product(choices, repeat=T):
            ids = np.array(combo, np.int32).reshape(T, k)
            offs, perm = oracle.dispatch(ids, E)
            bo, bp = _brute_dispatch(ids, E)
            assert np.array_equal(offs, bo) and np.array_equal(perm, bp)
            n += 1
    assert n == 1 + 8 + 216 + 1728 + 36


def test_dispatch_invariants_large():
    rng = np.random.default_rng(6)
    T, k, E = 5000, 8, 128
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    offs, perm = oracle.dispatch(ids, E)
    assert offs[0] == 0 and offs[-1] == T * k
    assert np.array_equal(np.sort(perm), np.arange(T * k))          # bijection
    assert np.array_equal(np.diff(offs), np.bincount(ids.reshape(-1), minlength=E))
    flat = ids.reshape(-1)
    for e in range(E):
        rows = perm[offs[e]:offs[e + 1]]
        assert np.all(flat[rows] == e) and np.all(np.diff(rows) > 0)  # ascending tokens


def test_planted_unstable_dispatch_is_caught():
    ids = np.array([[0, 1], [1, 0], [0, 2]], np.int32)
    offs, perm = oracle.dispatch(ids, 3)
    bo, bp = _brute_dispatch(ids, 3)
    assert np.array_equal(perm, bp)
    mutant = perm.copy()
    mutant[offs[0]:offs[1]] = mutant[offs[0]:offs[1]][::-1]  # tokens descending inside expert 0
    assert not np.array_equal(mutant, bp)


# ---------------------------------------------------------------- dequant
def test_dequant_int8_kat():
    q = np.array([[0x80, 0xFF, 0x00, 0x81]], np.uint8)
    s = np.array([0.5], np.float32)
    np.testing.assert_array_equal(oracle.dequant(q, s, "f32", 8, 0, 1, 4), [[0.0, 63.5, -64.0, 0.5]])


def test_dequant_int4_kat_low_nibble_first():
    q = np.array([[0x78, 0x0F]], np.uint8)  # bytes -> k0=8, k1=7, k2=15, k3=0
    s = np.array([2.0], np.float32)
    np.testing.assert_array_equal(oracle.dequant(q, s, "f32", 4, 0, 1, 4), [[0.0, -2.0, 14.0, -16.0]])


def test_planted_high_nibble_first_is_caught():
    q = np.array([[0x78]], np.uint8)
    s = np.array([1.0], np.float32)
    got = oracle.dequant(q, s, "f32", 4, 0, 1, 2)
    mutant = np.array([[(0x78 >> 4) - 8, (0x78 & 15) - 8]], np.float32)
    assert got.tolist() == [[0.0, -1.0]] and not np.array_equal(got, mutant)


@pytest.mark.parametrize("bits", [4, 8])
def test_dequant_block_scale_indexing(bits):
    K, bs = 64, 16
    nbytes = K // 2 if bits == 4 else K
    q = np.full((2, nbytes), 0x99 if bits == 4 else 0x81, np.uint8)  # every element decodes to +1
    s = (np.arange(2 * K // bs, dtype=np.float32) + 1).reshape(2, K // bs)
    got = oracle.dequant(q, s, "f32", bits, bs, 2, K)
    exp = np.repeat(s, bs, axis=1)
    np.testing.assert_array_equal(got, exp)


def test_dequant_f16_scales():
    q = np.array([[0x82]], np.uint8)
    s = np.array([0.1], np.float16)
    got = oracle.dequant(q, s, "f16", 8, 0, 1, 1)
    assert got[0, 0] == np.float32(2.0) * np.float32(np.float16(0.1))


# ---- quantizer round trip: the symmetric QMoE encoder as the benchmark
# configurations specify it (int8: s = max|w| / 127, q = clamp(round(w / s),
# -128, 127) + 128; int4: s = max|w| / 7, q = clamp(round(w / s), -8, 7) + 8,
# two per byte, even k in the low nibble; per output channel or per block
# along K), written here in float64 numpy with no code shared with the
# workload generator.  Decoding what it encodes must give back every weight
# to within half a quantisation step, and each row's (block's) largest
# magnitude exactly as +-127 s (+-7 s).  A decoder with another zero point or
# nibble order cannot meet that bound. ----
_SCALE_DT = {"f32": np.float32, "f16": np.float16}


def _store_scale(s64: np.ndarray, sdt: str):
    """float64 scales -> (stored array for the oracle, the stored values as float64)."""
    if sdt == "bf16":
        bits = oracle.f32_to_bf16_bits(s64.astype(np.float32))
        return bits, oracle.bf16_bits_to_f32(bits).astype(np.float64)
    st = s64.astype(_SCALE_DT[sdt])
    return st, st.astype(np.float64)


def _spec_quantize(w: np.ndarray, bits: int, block: int, sdt: str):
    """w [N, K] float32 -> (q uint8 [N, K*bits/8], stored scales, scales as float64 [N, K] broadcast)."""
    N, K = w.shape
    qmax = 127 if bits == 8 else 7
    bs = block if block else K
    wb = w.astype(np.float64).reshape(N, K // bs, bs)
    s_exact = np.abs(wb).max(axis=2) / qmax                          # [N, K/bs]
    s_store, s64 = _store_scale(s_exact if block else s_exact[:, 0], sdt)
    s_b = (s64 if block else s64[:, None]).reshape(N, K // bs, 1)
    v = np.clip(np.rint(wb / s_b), -qmax - 1, qmax).astype(np.int64).reshape(N, K)
    u = (v + (qmax + 1)).astype(np.uint8)                            # zero point 128 / 8
    q = u if bits == 8 else (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)
    return q, s_store, np.broadcast_to(s_b, (N, K // bs, bs)).reshape(N, K)


def _round_trip_excess(deq: np.ndarray, w: np.ndarray, s: np.ndarray) -> float:
    """max over elements of |deq - w| / (s / 2) (1 at the exact bound)."""
    return float(np.max(np.abs(deq.astype(np.float64) - w.astype(np.float64)) / (s / 2)))


ROUND_TRIP_CASES = [(bits, block, sdt) for bits in (8, 4) for block in (0, 16, 32, 128)
                    for sdt in ("f16", "bf16", "f32")]


@pytest.mark.parametrize("bits,block,sdt", ROUND_TRIP_CASES)
def test_quantizer_round_trip(bits, block, sdt):
    N, K = 24, 256
    rng = np.random.default_rng(100 + bits + block)
    w = (rng.standard_normal((N, K)) / math.sqrt(K)).astype(np.float32)
    # rows of different magnitude (scales stay fp16-normal: a subnormal
    # stored scale is coarser than the encoder's rounding step)
    w[3] *= np.float32(64.0)
    w[5] *= np.float32(0.25)
    q, s_store, s = _spec_quantize(w, bits, block, sdt)
    deq = oracle.dequant(q, s_store, sdt, bits, block, N, K)
    # every weight within half a step (plus the fp32 rounding of q * s)
    assert _round_trip_excess(deq, w, s) <= 1.0 + 1e-5
    # each row's / block's largest magnitude decodes to exactly +-qmax * s
    qmax = 127 if bits == 8 else 7
    bs = block if block else K
    wb = w.reshape(N, K // bs, bs)
    am = np.abs(wb).argmax(axis=2)
    peak = np.take_along_axis(deq.reshape(N, K // bs, bs), am[..., None], 2)[..., 0]
    sign = np.sign(np.take_along_axis(wb, am[..., None], 2)[..., 0])
    s_blk = s.reshape(N, K // bs, bs)[..., 0].astype(np.float32)
    np.testing.assert_array_equal(peak, sign * np.float32(qmax) * s_blk)


@pytest.mark.parametrize("bits,block", [(8, 0), (8, 32), (4, 32), (4, 128), (4, 0)])
def test_planted_encoding_mistakes_fail_round_trip(bits, block):
    """The decoder is planted with plausible mistakes by feeding it altered
    bytes or scales, which is what a decoder with that mistake would read:
    a zero point off by one (bytes - 1: every nibble / byte is >= 1 here),
    the high nibble first (nibbles swapped), and block scales taken along N
    instead of K (the scale array transposed).  Each must break the bound."""
    N, K = 16, 256
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((N, K)) / math.sqrt(K)).astype(np.float32)
    q, s_store, s = _spec_quantize(w, bits, block, "f32")
    good = oracle.dequant(q, s_store, "f32", bits, block, N, K)
    assert _round_trip_excess(good, w, s) <= 1.0 + 1e-5
    mutants = {"zero point off by one": (q - (0x11 if bits == 4 else 1)).astype(np.uint8)}
    if bits == 4:
        mutants["high nibble first"] = (((q & 0x0F) << 4) | (q >> 4)).astype(np.uint8)
    for what, qm in mutants.items():
        bad = oracle.dequant(qm, s_store, "f32", bits, block, N, K)
        assert _round_trip_excess(bad, w, s) > 1.5, what
    if block:
        st = np.ascontiguousarray(s_store.reshape(N, K // block).T).reshape(N, K // block)
        bad = oracle.dequant(q, st, "f32", bits, block, N, K)
        assert _round_trip_excess(bad, w, s) > 1.5, "block scales along N"


# ---------------------------------------------------------------- MXFP4
# OCP Microscaling Formats (MX) v1.0: FP4 E2M1 elements (1 sign, 2 exponent
# bits with bias 1, 1 mantissa bit), E8M0 block scales of 32 elements.
E2M1_GRID = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def test_e2m1_and_e8m0_known_answers():
    lib = oracle.load()
    got = [lib.orc_e2m1_to_f32(n) for n in range(16)]
    assert got[:8] == list(E2M1_GRID)
    assert got[8:] == list(-E2M1_GRID)
    assert math.copysign(1.0, got[8]) == -1.0                  # 0b1000 is -0
    for e, v in ((127, 1.0), (128, 2.0), (126, 0.5), (0, 2.0 ** -127), (254, 2.0 ** 127), (137, 1024.0)):
        assert lib.orc_e8m0_to_f32(e) == v, e
    assert math.isnan(lib.orc_e8m0_to_f32(255))


def test_mxfp4_hand_packed_bytes():
    """One row, K = 64: two scale blocks.  Even k is the low nibble."""
    q = np.zeros((1, 32), np.uint8)
    q[0, 0] = 0x2F          # k0 = -6 (0xF), k1 = +1 (0x2)
    q[0, 1] = 0x90          # k2 = 0, k3 = -0.5 (0x9)
    q[0, 16] = 0x71         # k32 = 0.5, k33 = 6
    s = np.array([[128, 125]], np.uint8)                       # 2 and 1/4
    d = oracle.dequant_mxfp4(q, s, 1, 64)[0]
    assert list(d[:4]) == [-12.0, 2.0, 0.0, -1.0]
    assert list(d[32:34]) == [0.125, 1.5]
    assert not d[4:32].any() and not d[34:].any()
    nan = oracle.dequant_mxfp4(q, np.array([[255, 127]], np.uint8), 1, 64)[0]
    assert np.isnan(nan[:32]).all() and list(nan[32:34]) == [0.5, 6.0]


def _spec_quantize_mxfp4(w: np.ndarray):
    """The MX v1.0 quantizer (section 6.3): shared exponent
    floor(log2(max|w|)) - 2 (E2M1's largest exponent), elements rounded to the
    nearest E2M1 value (ties to the even mantissa) and clamped to +-6."""
    N, K = w.shape
    wb = w.astype(np.float64).reshape(N, K // 32, 32)
    amax = np.abs(wb).max(axis=2)
    e = np.where(amax > 0, np.floor(np.log2(np.where(amax > 0, amax, 1))) - 2, -127).astype(np.int64)
    X = np.ldexp(1.0, e)[:, :, None]
    a = np.minimum(np.abs(wb) / X, 6.0)
    dist = np.abs(a[..., None] - E2M1_GRID)                    # nearest grid point; ties -> even code
    best = dist.min(-1, keepdims=True)
    cand = np.where(dist == best, np.arange(8), 99)
    even = np.where(cand % 2 == 0, cand, 99).min(-1)
    code = np.where(even < 99, even, cand.min(-1))
    nib = (code | np.where(wb < 0, 8, 0)).reshape(N, K).astype(np.uint8)
    q = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    return q, (e + 127).astype(np.uint8), np.broadcast_to(X, wb.shape).reshape(N, K)


def _mxfp4_excess(d: np.ndarray, w: np.ndarray, X: np.ndarray) -> float:
    """max |d - w| over the nearest-value bound: half the grid step at |w|/X
    (0.25, 0.5, 1 for [0,2), [2,4), [4,6]) and the clamp distance past 6."""
    a = np.abs(w.astype(np.float64)) / X
    half = np.where(a < 2, 0.25, np.where(a < 4, 0.5, 1.0))
    bound = np.maximum(half, a - 6.0) * X
    return float(np.max(np.abs(d.astype(np.float64) - w) / bound))


def test_mxfp4_quantizer_round_trip_and_planted_mistakes():
    N, K = 16, 256
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((N, K)) * np.array([1e-3, 1.0, 40.0, 3e4])[rng.integers(0, 4, (N, 1))]).astype(np.float32)
    q, s, X = _spec_quantize_mxfp4(w)
    good = oracle.dequant_mxfp4(q, s, N, K)
    assert _mxfp4_excess(good, w, X) <= 1.0 + 1e-9
    # each block's largest element lands in [4, 6] x X, the top binade
    top = np.abs(good.reshape(N, K // 32, 32)).max(2) / X.reshape(N, K // 32, 32)[:, :, 0]
    assert ((top >= 4) & (top <= 6)).all()
    mutants = {"high nibble first": (((q & 0x0F) << 4) | (q >> 4)).astype(np.uint8),
               "sign bit as mantissa": (q ^ 0x99).astype(np.uint8)}
    for what, qm in mutants.items():
        assert _mxfp4_excess(oracle.dequant_mxfp4(qm, s, N, K), w, X) > 1.5, what
    assert _mxfp4_excess(oracle.dequant_mxfp4(q, (s + 1).astype(np.uint8), N, K), w, X) > 1.5, "scale bias 126"
    assert _mxfp4_excess(oracle.dequant_mxfp4(q, (s - 1).astype(np.uint8), N, K), w, X) > 1.5, "scale bias 128"


def test_workload_mxfp4_quantizer_matches_spec():
    """The benchmark's torch MXFP4 encoder produces the spec quantizer's bytes
    (including ties, zero blocks and saturation)."""
    import torch
    from onnxruntime_musa_amd.workloads import quantize_mxfp4
    rng = np.random.default_rng(21)
    w = (rng.standard_normal((8, 128)) * 3).astype(np.float32)
    w[0, :32] = 0.0                                                # zero block
    w[1, :32] = np.float32([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0] * 4)  # ties at X = 1 (amax 6)
    w[2, :32] = np.float32(2.0 ** np.arange(-16, 16))              # a wide block: small values round to 0
    q, s = quantize_mxfp4(torch.from_numpy(w))
    q_ref, s_ref, _ = _spec_quantize_mxfp4(w)
    np.testing.assert_array_equal(q.numpy(), q_ref)
    np.testing.assert_array_equal(s.numpy(), s_ref)


def test_mxfp4_forward_matches_float64_formulation():
    """The forward with MXFP4 experts against a dense float64 restatement that
    decodes with numpy's own table (E2M1_GRID, 2.0 ** (s - 127))."""
    T, H, I, E, k = 12, 64, 32, 4, 2
    rng = np.random.default_rng(5)
    x = rng.standard_normal((T, H)).astype(np.float32)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    q1, s1, _ = zip(*[_spec_quantize_mxfp4(rng.standard_normal((2 * I, H)).astype(np.float32) / 8) for _ in range(E)])
    q2, s2, _ = zip(*[_spec_quantize_mxfp4(rng.standard_normal((H, I)).astype(np.float32) / 8) for _ in range(E)])
    q1, s1, q2, s2 = map(np.stack, (q1, s1, q2, s2))
    b1 = rng.standard_normal((E, 2 * I)).astype(np.float32)
    b2 = rng.standard_normal((E, H)).astype(np.float32)
    r = oracle.moe_forward(x=x, logits=lg, w1=q1, w2=q2, k=k, hidden=H, inter=I, experts=E, activation="swiglu",
                           swiglu_fusion=1, swiglu_limit=7.0, alpha=1.702, beta=1.0, normalize=1, bits=4,
                           block_size=32, scale_dtype="f32", s1=s1, b1=b1, s2=s2, b2=b2, weight_format=1)

    def deq(qe, se):
        nib = np.stack([qe & 0x0F, qe >> 4], -1).reshape(qe.shape[0], -1)
        val = np.where(nib & 8, -1.0, 1.0) * E2M1_GRID[nib & 7]
        return val * np.repeat(2.0 ** (se.astype(np.float64) - 127), 32, axis=1)

    p = np.exp(lg - lg.max(1, keepdims=True))
    order = np.argsort(-lg, axis=1, kind="stable")[:, :k]
    wsel = np.take_along_axis(p, order, 1)
    wsel /= wsel.sum(1, keepdims=True)
    ref = np.zeros((T, H))
    for e in range(E):
        tok, slot = np.nonzero(order == e)
        h1 = x[tok].astype(np.float64) @ deq(q1[e], s1[e]).T + b1[e]
        g, l = np.minimum(h1[:, 0::2], 7.0), np.clip(h1[:, 1::2], -7.0, 7.0)
        a = g / (1 + np.exp(-1.702 * g)) * (l + 1.0)
        y = a @ deq(q2[e], s2[e]).T + b2[e]
        ref[tok] += wsel[tok, slot][:, None] * y
    np.testing.assert_allclose(r["out_f32"], ref, rtol=1e-5, atol=1e-5)
    with pytest.raises(ValueError):
        oracle.moe_forward(x=x, logits=lg, w1=q1, w2=q2, k=k, hidden=H, inter=I, experts=E, activation="swiglu",
                           swiglu_fusion=1, bits=4, block_size=16, scale_dtype="f32", s1=s1, s2=s2, weight_format=1)


# ---------------------------------------------------------------- activations
def test_activation_closed_forms():
    h = np.array([1.0, -2.0, 0.5], np.float32)
    np.testing.assert_allclose(oracle.activation(h, None, 3, "silu"), h / (1 + np.exp(-h)), rtol=1e-6)
    erf = np.vectorize(math.erf)
    np.testing.assert_allclose(oracle.activation(h, None, 3, "gelu"), 0.5 * h * (1 + erf(h / math.sqrt(2))),
                               rtol=1e-6)
    np.testing.assert_array_equal(oracle.activation(h, None, 3, "relu"), [1.0, 0.0, 0.5])
    np.testing.assert_array_equal(oracle.activation(h, None, 3, "identity"), h)
    assert abs(oracle.activation(np.array([1.0], np.float32), None, 1, "silu")[0] - 0.7310585786300049) < 1e-7


def test_swiglu_layouts_and_clamp():
    g = np.array([10.0, -1.0], np.float32)
    l = np.array([-10.0, 2.0], np.float32)
    alpha, beta, lim = 1.702, 1.0, 7.0

    def ref(g, l):
        G = np.minimum(g, lim)
        L = np.clip(l, -lim, lim)
        return G / (1 + np.exp(-alpha * G)) * (L + beta)

    inter = np.stack([g, l], 1).reshape(-1)
    chunk = np.concatenate([g, l])
    np.testing.assert_allclose(oracle.activation(inter, None, 2, "swiglu", 1, alpha, beta, lim), ref(g, l), rtol=1e-6)
    np.testing.assert_allclose(oracle.activation(chunk, None, 2, "swiglu", 2, alpha, beta, lim), ref(g, l), rtol=1e-6)
    np.testing.assert_allclose(oracle.activation(g, l, 2, "swiglu", 0, alpha, beta, lim), ref(g, l), rtol=1e-6)
    # SiLU gating with fc3
    np.testing.assert_allclose(oracle.activation(g, l, 2, "silu"), g / (1 + np.exp(-g)) * l, rtol=1e-6)


def _silu64(g):
    g = np.asarray(g, np.float64)
    return g / (1.0 + np.exp(-g))


def test_swiglu_reduces_to_textbook_swish_glu():
    """alpha = 1, beta = 0, no limit: SwiGLU(g, l) = Swish_1(g) * l, the GLU
    variant of Shazeer, "GLU Variants Improve Transformer" (2020), eq. 6."""
    rng = np.random.default_rng(11)
    g = (rng.standard_normal(64) * 4).astype(np.float32)
    l = (rng.standard_normal(64) * 4).astype(np.float32)
    exp = _silu64(g) * l.astype(np.float64)
    for fusion, h1, h3 in [(0, g, l), (1, np.stack([g, l], 1).reshape(-1), None), (2, np.concatenate([g, l]), None)]:
        got = oracle.activation(h1, h3, 64, "swiglu", fusion, 1.0, 0.0, float("inf"))
        np.testing.assert_allclose(got, exp, rtol=2e-6, atol=1e-7)


def test_swiglu_large_alpha_gates_like_relu():
    """sigma(alpha g) tends to the step function as alpha grows, so
    g * sigma(alpha g) * (l + beta) tends to relu(g) * (l + beta)."""
    g = np.array([-3.0, -0.5, 0.5, 3.0], np.float32)
    l = np.array([1.5, -2.0, 0.25, -0.75], np.float32)
    got = oracle.activation(g, l, 4, "swiglu", 0, 1e4, 1.0, float("inf"))
    np.testing.assert_allclose(got, np.maximum(g, 0) * (l + 1.0), rtol=1e-6, atol=1e-30)


def test_swiglu_clamp_saturation():
    """With a limit: a gate at or above it gives the same output whatever its
    value (one-sided: a gate below -limit is not clamped), a linear input is
    clamped on both sides, and beta is added after the clamp (the form of
    the published gpt-oss SwiGLU, openai/gpt-oss, which this config mirrors)."""
    lim, alpha, beta = 7.0, 1.702, 1.0

    def one(g, l):
        return float(oracle.activation(np.array([g], np.float32), np.array([l], np.float32), 1, "swiglu", 0,
                                       alpha, beta, lim)[0])

    at = one(lim, 0.5)
    for g in (7.25, 50.0, 1e30, np.inf):
        assert one(g, 0.5) == at
    assert one(-7.5, 0.5) != one(-8.0, 0.5)                # no clamp below -limit for the gate
    assert one(2.0, 9.0) == one(2.0, lim) and one(2.0, -40.0) == one(2.0, -lim)
    assert one(2.0, 6.0) != one(2.0, lim)                  # below the limit nothing is clamped
    # beta after the clamp: l = 6.5 gives (6.5 + 1), not clamp(7.5) = 7
    np.testing.assert_allclose(one(2.0, 6.5), float(2.0 / (1 + np.exp(-alpha * 2.0)) * 7.5), rtol=1e-6)
    # and beta is a shift of the linear input below the limit
    assert one(2.0, 3.0) == float(oracle.activation(np.array([2.0], np.float32), np.array([4.0], np.float32), 1,
                                                    "swiglu", 0, alpha, 0.0, lim)[0])


def test_planted_swapped_gate_linear_is_caught():
    g = np.array([3.0], np.float32)
    l = np.array([-0.5], np.float32)
    good = oracle.activation(np.array([3.0, -0.5], np.float32), None, 1, "swiglu", 1)
    swapped = oracle.activation(np.array([-0.5, 3.0], np.float32), None, 1, "swiglu", 1)
    assert np.isclose(good[0], 3.0 / (1 + math.exp(-3.0)) * -0.5) and not np.isclose(good[0], swapped[0])


# ---------------------------------------------------------------- forward
def _np64_forward(cfg, h):
    """Independent float64 formulation with dense matmuls over all tokens."""
    T = h["input"].shape[0]
    x = oracle.to_f32(h["input"], cfg.dtype).astype(np.float64)
    lg = oracle.to_f32(h["router_probs"], cfg.dtype).astype(np.float64)
    p = np.exp(lg - lg.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    order = np.argsort(-lg, axis=1, kind="stable")[:, :cfg.k]
    w = np.take_along_axis(p, order, 1)
    if cfg.normalize:
        w /= w.sum(1, keepdims=True)

    def mat(name, sname, N, K):
        q = h.get(name)
        if q is None:
            return None
        if cfg.bits == 0:
            return oracle.to_f32(q, cfg.dtype).astype(np.float64)
        return np.stack([oracle.dequant(q[e], h[sname][e], cfg.scale_dtype, cfg.bits, cfg.block_size, N, K)
                         for e in range(cfg.experts)]).astype(np.float64)

    def vec(name):
        return None if h.get(name) is None else oracle.to_f32(h[name], cfg.dtype).astype(np.float64)

    W1 = mat("fc1_experts_weights", "fc1_scales", cfg.n1, cfg.hidden)
    W2 = mat("fc2_experts_weights", "fc2_scales", cfg.hidden, cfg.inter)
    W3 = mat("fc3_experts_weights", "fc3_scales", cfg.inter, cfg.hidden)
    b1, b2, b3 = vec("fc1_experts_bias"), vec("fc2_experts_bias"), vec("fc3_experts_bias")
    sig = lambda v: 1 / (1 + np.exp(-v))  # noqa: E731
    lim = np.inf if cfg.swiglu_limit is None else cfg.swiglu_limit
    out = np.zeros((T, cfg.hidden))
    for e in range(cfg.experts):
        tok, slot = np.nonzero(order == e)
        if tok.size == 0:
            continue
        h1 = x[tok] @ W1[e].T + (0 if b1 is None else b1[e])
        if W3 is not None:
            h3 = x[tok] @ W3[e].T + (0 if b3 is None else b3[e])
            g, l = h1, h3
        elif cfg.activation == "swiglu":
            g, l = (h1[:, 0::2], h1[:, 1::2]) if cfg.swiglu_fusion == 1 else (h1[:, :cfg.inter], h1[:, cfg.inter:])
        else:
            g, l = h1, None
        if cfg.activation == "swiglu":
            G = np.minimum(g, lim)
            a = G * sig(cfg.alpha * G) * (np.clip(l, -lim, lim) + cfg.beta)
        else:
            a = {"silu": g * sig(g), "relu": np.maximum(g, 0), "identity": g}[cfg.activation]
            if l is not None:
                a = a * l
        y = a @ W2[e].T + (0 if b2 is None else b2[e])
        out[tok] += w[tok, slot][:, None] * y
    return out


def _problem(name, T=24, seed=1, **over):
    from onnxruntime_musa_amd.workloads import CONFIGS, make_problem, to_host
    p = make_problem(CONFIGS[name], T, seed=seed, device="cpu", gen="numpy", **over)
    return p.cfg, {n: to_host(t) for n, t in p.inputs.items()}


FORWARD_CASES = [
    ("c1_moe_f32", {}),
    ("c2_qmoe_int8_mixtral", dict(hidden=128, inter=256)),
    ("c3_qmoe_int4_mixtral", dict(hidden=128, inter=256)),
    ("c4_qmoe_int4_gptoss", dict(hidden=128, inter=192, experts=8)),
    ("c5_moe_f16_qwen3", dict(hidden=128, inter=64, experts=16, k=4)),
    ("c3_qmoe_int4_mixtral", dict(hidden=128, inter=256, use_fc3=False, swiglu_fusion=2, bias=True)),
    ("c1_moe_f32", dict(activation="relu", normalize=0)),
    ("c1_moe_f32", dict(activation="silu", use_fc3=True, bias=True)),
]


@pytest.mark.parametrize("name,over", FORWARD_CASES)
def test_forward_matches_float64_formulation(name, over):
    cfg, h = _problem(name, **over)
    r = oracle.forward_problem(cfg, h)
    ref = _np64_forward(cfg, h)
    np.testing.assert_allclose(r["out_f32"], ref, rtol=1e-5, atol=2e-6)


def test_planted_dropped_bias_is_caught():
    cfg, h = _problem("c1_moe_f32")
    ref = _np64_forward(cfg, h)
    h2 = dict(h)
    h2["fc2_experts_bias"] = None
    bad = oracle.forward_problem(cfg, h2)["out_f32"]
    assert np.max(np.abs(bad - ref)) > 1e-3


def test_unfused_equals_fused_layouts():
    from dataclasses import replace
    cfg, h = _problem("c1_moe_f32", activation="swiglu", use_fc3=True, bias=True)
    base = oracle.forward_problem(cfg, h)["out_f32"]
    W1, W3 = h["fc1_experts_weights"], h["fc3_experts_weights"]
    b1, b3 = h["fc1_experts_bias"], h["fc3_experts_bias"]
    chunk = dict(h, fc1_experts_weights=np.concatenate([W1, W3], 1), fc1_experts_bias=np.concatenate([b1, b3], 1),
                 fc3_experts_weights=None, fc3_experts_bias=None)
    inter_w = np.stack([W1, W3], 2).reshape(W1.shape[0], -1, W1.shape[2])
    inter_b = np.stack([b1, b3], 2).reshape(b1.shape[0], -1)
    inter = dict(chunk, fc1_experts_weights=inter_w, fc1_experts_bias=inter_b)
    c2 = oracle.forward_problem(replace(cfg, use_fc3=False, swiglu_fusion=2), chunk)["out_f32"]
    c1 = oracle.forward_problem(replace(cfg, use_fc3=False, swiglu_fusion=1), inter)["out_f32"]
    np.testing.assert_array_equal(base, c2)
    np.testing.assert_array_equal(base, c1)


@pytest.mark.parametrize("name", ["c2_qmoe_int8_mixtral", "c3_qmoe_int4_mixtral"])
def test_qmoe_equals_moe_on_dequantised_weights(name):
    from dataclasses import replace
    cfg, h = _problem(name, hidden=128, inter=256, dtype="f32", scale_dtype="f32")
    q = oracle.forward_problem(cfg, h)["out_f32"]
    deq = {}
    for w, s, N, K in [("fc1_experts_weights", "fc1_scales", cfg.n1, cfg.hidden),
                       ("fc2_experts_weights", "fc2_scales", cfg.hidden, cfg.inter),
                       ("fc3_experts_weights", "fc3_scales", cfg.inter, cfg.hidden)]:
        deq[w] = np.stack([oracle.dequant(h[w][e], h[s][e], "f32", cfg.bits, cfg.block_size, N, K)
                           for e in range(cfg.experts)])
    dense = {n: v for n, v in h.items() if not n.endswith("scales")}
    dense.update(deq)
    m = oracle.forward_problem(replace(cfg, bits=0, block_size=0), dense)["out_f32"]
    np.testing.assert_array_equal(q, m)


def test_single_expert_is_dense_ffn():
    cfg, h = _problem("c1_moe_f32", experts=1, k=1, activation="silu")
    r = oracle.forward_problem(cfg, h)
    x = h["input"].astype(np.float64)
    a = x @ h["fc1_experts_weights"][0].T.astype(np.float64) + h["fc1_experts_bias"][0]
    a = a / (1 + np.exp(-a))
    y = a @ h["fc2_experts_weights"][0].T.astype(np.float64) + h["fc2_experts_bias"][0]
    np.testing.assert_allclose(r["out_f32"], y, rtol=1e-5, atol=2e-6)
    assert np.all(r["topk_w"] == 1.0)


def test_linear_in_fc2_scales():
    cfg, h = _problem("c2_qmoe_int8_mixtral", hidden=128, inter=128, dtype="f32", scale_dtype="f32")
    a = oracle.forward_problem(cfg, h)["out_f32"]
    h2 = dict(h, fc2_scales=h["fc2_scales"] * np.float32(2.0))
    b = oracle.forward_problem(cfg, h2)["out_f32"]
    np.testing.assert_allclose(b, 2 * a, rtol=1e-6, atol=1e-7)


def test_token_mask_computes_only_masked_rows():
    cfg, h = _problem("c1_moe_f32", T=20)
    full = oracle.forward_problem(cfg, h)["out_f32"]
    mask = np.zeros(20, np.uint8)
    mask[[3, 7, 19]] = 1
    part = oracle.forward_problem(cfg, h, token_mask=mask)["out_f32"]
    np.testing.assert_array_equal(part[[3, 7, 19]], full[[3, 7, 19]])


def test_thread_count_does_not_change_results():
    cfg, h = _problem("c3_qmoe_int4_mixtral", hidden=128, inter=256)
    a = oracle.forward_problem(cfg, h, threads=1)["out_f32"]
    b = oracle.forward_problem(cfg, h, threads=4)["out_f32"]
    np.testing.assert_array_equal(a, b)


# ---------------------------------------------------------------- fixtures
def test_golden_c1_fixture():
    """configs[0] (fp32 MoE, 64 tokens) from its seed: oracle output and routing
    equal the committed fixture."""
    fx = np.load(GOLDEN / "c1_moe_f32_seed0.npz", allow_pickle=False)
    cfg, h = _problem("c1_moe_f32", T=int(fx["tokens"]), seed=int(fx["seed"]))
    np.testing.assert_array_equal(h["input"].reshape(-1)[:16], fx["input_head"])
    r = oracle.forward_problem(cfg, h)
    np.testing.assert_array_equal(r["topk_ids"], fx["topk_ids"])
    np.testing.assert_array_equal(r["perm"], fx["perm"])
    np.testing.assert_allclose(r["out_f32"], fx["out"], rtol=0, atol=1e-6)


@pytest.mark.parametrize("fixture", sorted(p.name for p in GOLDEN.glob("qmoe_*.npz")))
def test_golden_qmoe_fixtures(fixture):
    from onnxruntime_musa_amd.workloads import CONFIGS
    fx = np.load(GOLDEN / fixture, allow_pickle=False)
    name = str(fx["config"])
    over = {k: int(fx[k]) for k in ("hidden", "inter", "experts")}
    cfg, h = _problem(name, T=int(fx["tokens"]), seed=int(fx["seed"]), **over)
    assert cfg.bits == CONFIGS[name].bits
    r = oracle.forward_problem(cfg, h)
    np.testing.assert_array_equal(r["topk_ids"], fx["topk_ids"])
    np.testing.assert_allclose(r["out_f32"], fx["out"], rtol=0, atol=1e-6)


# ---- TopK restatement (oracle.topk), pinned by the known answers the
# reference's TopK tests state (test/ops/test_topk.py) ----
def test_topk_oracle_reference_known_answers():
    # :195-209 integers above 2^53 are ordered exactly
    v, i = oracle.topk(np.array([[2**53, 2**53 + 1, 2**53 + 2, 0]], dtype=np.int64), 2)
    np.testing.assert_array_equal(v, [[2**53 + 2, 2**53 + 1]])
    np.testing.assert_array_equal(i, [[2, 1]])
    # :212-227 adjacent float32 values are not ties
    nxt = np.nextafter(np.float32(10.0), np.float32(np.inf))
    v, i = oracle.topk(np.array([[10.0, nxt, 9.0]], dtype=np.float32), 1)
    assert v[0, 0] == nxt and i[0, 0] == 1
    # :230-246 k = 1 along a non-last axis, smallest, ties -> lower index
    x = np.array([[[4.0, 7.0], [1.0, 7.0], [1.0, 8.0], [3.0, 9.0]]], dtype=np.float32)
    v, i = oracle.topk(x, 1, axis=1, largest=0)
    np.testing.assert_array_equal(v, [[[1.0, 7.0]]])
    np.testing.assert_array_equal(i, [[[1, 0]]])
    # :307-323 all equal -> arange(k), both directions
    for largest in (0, 1):
        v, i = oracle.topk(np.full((1, 4000), 3.25, dtype=np.float32), 128, largest=largest)
        np.testing.assert_array_equal(i, np.arange(128)[None, :])
    # :291-304 k = 0 gives empty outputs
    v, i = oracle.topk(np.array([[3.0, 1.0, 2.0], [6.0, 5.0, 4.0]], dtype=np.float32), 0)
    assert v.shape == (2, 0) and i.shape == (2, 0)


def test_topk_oracle_against_stable_sort_and_brute_force():
    rng = np.random.default_rng(3)
    for trial in range(20):
        d = int(rng.integers(1, 40))
        x = rng.integers(-4, 5, size=(3, d)).astype(np.float32)  # many ties
        k = int(rng.integers(0, d + 1))
        for largest in (0, 1):
            v, i = oracle.topk(x, k, largest=largest)
            key = -x if largest else x
            order = np.argsort(key, axis=-1, kind="stable")[:, :k]
            np.testing.assert_array_equal(i, order)
            np.testing.assert_array_equal(v, np.take_along_axis(x, order, axis=-1))
    # -0.0 ties with +0.0 (value comparison): the lower index comes first
    v, i = oracle.topk(np.array([[0.0, -0.0, 0.0]], dtype=np.float32), 3)
    np.testing.assert_array_equal(i, [[0, 1, 2]])
    # a planted mistake (ties toward the higher index) is caught
    x = np.array([[1.0, 2.0, 2.0, 0.0]], dtype=np.float32)
    _, i = oracle.topk(x, 1)
    assert i[0, 0] == 1 and i[0, 0] != 2


def test_softmax_oracle_closed_forms():
    # rows sum to one; uniform rows give 1/dim; shift invariance; two-element
    # softmax is the logistic function of the difference
    rng = np.random.default_rng(4)
    x = rng.standard_normal((5, 7, 3))
    for axis in (0, 1, 2, -1):
        y = oracle.softmax(x, axis)
        np.testing.assert_allclose(np.sum(y, axis=axis), 1.0, rtol=1e-12)
        np.testing.assert_allclose(oracle.softmax(x + 123.0, axis), y, rtol=1e-12)
    np.testing.assert_allclose(oracle.softmax(np.zeros((2, 8)), -1), 1.0 / 8)
    a, b = 0.7, -1.9
    y = oracle.softmax(np.array([[a, b]]), -1)
    np.testing.assert_allclose(y[0, 0], 1.0 / (1.0 + np.exp(b - a)), rtol=1e-14)
    # the router's softmax (the C oracle) on the same logits agrees
    lg = rng.standard_normal((6, 8)).astype(np.float32)
    _, w = oracle.route(lg, 8, False, False)
    ids, _ = oracle.route(lg, 8, False, False)
    np.testing.assert_allclose(w, np.take_along_axis(oracle.softmax(lg.astype(np.float64), -1), ids, axis=-1),
                               rtol=1e-5)


# ---- router GEMM restatement (oracle.gate_logits): a float64 matmul
# rounded once to the activation type, pinned by exact integer arithmetic and
# by the rounding of the types ----
@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_gate_logits_exact_integer_products(dtype):
    rng = np.random.default_rng(21)
    T, H, E = 7, 96, 9
    xi = rng.integers(-3, 4, size=(T, H))
    wi = rng.integers(-4, 5, size=(E, H))
    bi = rng.integers(-5, 6, size=E)
    cast = {"f32": lambda a: a.astype(np.float32), "f16": lambda a: a.astype(np.float16),
            "bf16": lambda a: oracle.f32_to_bf16_bits(a.astype(np.float32))}[dtype]
    got = oracle.to_f32(oracle.gate_logits(cast(xi), cast(wi), cast(bi), dtype), dtype)
    exact = (xi @ wi.T + bi).astype(np.float64)          # integers below 2^8: exact in every type
    np.testing.assert_array_equal(got.astype(np.float64), exact)


def test_gate_logits_round_once():
    # a value between two bf16 neighbours rounds to the nearer one, a tie to even
    x = oracle.f32_to_bf16_bits(np.array([[1.0, 1.0]], np.float32))
    w = oracle.f32_to_bf16_bits(np.array([[1.0, 2.0 ** -8], [1.0, 3 * 2.0 ** -9]], np.float32))
    got = oracle.to_f32(oracle.gate_logits(x, w, None, "bf16"), "bf16")
    # 1 + 2^-8 is halfway between 1 and 1 + 2^-7: ties to even (1); 1 + 3 2^-9 rounds up
    np.testing.assert_array_equal(got, [[1.0, 1.0 + 2.0 ** -7]])
    # a planted double rounding (float64 -> float32 -> bf16 without care) is not what the oracle does
    assert oracle.f64_to_bf16_bits(np.array([1.0 + 2.0 ** -8 + 2.0 ** -40]))[0] == 0x3F81
