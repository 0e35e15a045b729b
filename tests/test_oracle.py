"""CPU checks that pin the oracle before anything is compared against it.

Each check is chosen so a plausible mistake in the restatement fails it:
hand-packed words catch a wrong nibble order, closed forms catch a dropped
scale or bias, exact integer cases catch rounding slips, the independent numpy
and fp64 restatements catch accumulation or indexing errors, and reductions
(one-hot x, E=1 gather, linearity) catch transposed operands.
"""
import json
import os

import numpy as np
import pytest

from synth import deq_numpy, make_quant, make_x, pack, rel_err, unpack

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------- bf16 / packing

def test_bf16_round_to_nearest_even(oracle):
    f = np.array([1.0, 1.00390625, 1.005859375, 1.0078125, 1.01171875, -2.5, 3.0e38, 1e-40],
                 dtype=np.float32)
    # 1 + 2^-8 is a tie -> even (1.0); 1 + 1.5*2^-8 rounds up to 1 + 2^-7
    want = [0x3F80, 0x3F80, 0x3F81, 0x3F81, 0x3F82, 0xC020, 0x7F62, 0x0001]
    got = oracle.f32_to_bf16(f)
    assert [int(v) for v in got] == want
    for v, w in zip(f, want):
        assert oracle.lib().oracle_f32_to_bf16(float(v)) == w
    assert oracle.f32_to_bf16(np.array([np.nan], dtype=np.float32))[0] & 0x7FFF > 0x7F80


def test_pack_order_lsb_first(oracle):
    # element k of a row sits at bit (k % 8) * 4 of word k / 8
    w = np.array([[0x76543210, 0xFEDCBA98]], dtype=np.uint32)
    assert unpack(w, 4).tolist() == [list(range(16))]
    assert [oracle.lib().oracle_unpack(w.ctypes.data_as(__import__("ctypes").c_void_p), k, 4)
            for k in range(16)] == list(range(16))
    w8 = np.array([[0x03020100, 0xFFFEFDFC]], dtype=np.uint32)
    assert unpack(w8, 8).tolist() == [[0, 1, 2, 3, 0xFC, 0xFD, 0xFE, 0xFF]]
    q = np.arange(64, dtype=np.uint32).reshape(1, 64) % 16
    assert np.array_equal(unpack(pack(q, 4), 4), q)


def _lib_unpack_sig(oracle):
    import ctypes
    L = oracle.lib()
    L.oracle_unpack.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int]
    L.oracle_unpack.restype = ctypes.c_uint32


@pytest.fixture(autouse=True)
def _sig(oracle):
    _lib_unpack_sig(oracle)


# ---------------------------------------------------------------- dequantize

def test_dequant_closed_forms(oracle):
    # s = 1, b = 0: dequant returns q exactly
    K = 64
    q = (np.arange(K, dtype=np.uint32) % 16).reshape(1, K)
    w = pack(q, 4)
    one = np.array([[0x3F80]], dtype=np.uint16)
    zero = np.array([[0x0000]], dtype=np.uint16)
    out = oracle.bf16_to_f32(oracle.dequantize(w, one, zero, 64, 4))
    assert out.tolist() == [q[0].astype(np.float32).tolist()]
    # s = 0.5, b = -4: q/2 - 4, exact in bf16
    half = np.array([[0x3F00]], dtype=np.uint16)
    m4 = np.array([[0xC080]], dtype=np.uint16)
    out = oracle.bf16_to_f32(oracle.dequantize(w, half, m4, 64, 4))
    assert out.tolist() == [(q[0] * 0.5 - 4).astype(np.float32).tolist()]
    # q = 0 -> b; s = 0 -> b
    rng = np.random.default_rng(0)
    w0, s0, b0 = make_quant(rng, (8,), 128, 4, 64)
    zq = np.zeros_like(w0)
    out = oracle.dequantize(zq, s0, b0, 64, 4)
    assert np.array_equal(out, np.repeat(b0, 64, axis=1))
    out = oracle.dequantize(w0, np.zeros_like(s0), b0, 64, 4)
    assert np.array_equal(out, np.repeat(b0, 64, axis=1))


def test_dequant_double_rounding_is_observable(oracle):
    """The two rounding sequences differ on a hand-built case, so the choice matters.

    s = 1 + 2^-7 (bf16 0x3F81), q = 3: q*s = 3.0234375 -> bf16 3.03125 (tie to even up);
    b = 2^-6: bf16(3.03125 + 0.015625) = 3.046875, while one rounding of
    3.0234375 + 0.015625 = 3.0390625 gives 3.03125 (tie to even down)."""
    w = pack(np.array([[3] + [0] * 63], dtype=np.uint32), 4)
    s = np.array([[0x3F81]], dtype=np.uint16)
    b = np.array([[0x3C80]], dtype=np.uint16)
    mlx = oracle.bf16_to_f32(oracle.dequantize(w, s, b, 64, 4, oracle.DEQ_MLX))[0, 0]
    fused = oracle.bf16_to_f32(oracle.dequantize(w, s, b, 64, 4, oracle.DEQ_FUSED))[0, 0]
    assert mlx == np.float32(3.046875)
    assert fused == np.float32(3.03125)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_dequant_matches_independent_numpy(oracle, bits, group):
    rng = np.random.default_rng(bits * group)
    w, s, b = make_quant(rng, (33,), 512, bits, group)
    for fused, mode in ((False, oracle.DEQ_MLX), (True, oracle.DEQ_FUSED)):
        ref = deq_numpy(w, s, b, bits, group, fused=fused)
        got = oracle.bf16_to_f32(oracle.dequantize(w, s, b, group, bits, mode))
        assert np.array_equal(got, ref)


def test_dequant_vs_fp64_brute_force(oracle):
    """All q against a sweep of bf16 scales/biases: the MLX sequence is within two
    half-ulps of the exact value s*q + b -- one relative to q*s (first rounding),
    one relative to the result (second rounding)."""
    rng = np.random.default_rng(9)
    pats = rng.integers(0x3000, 0x4200, size=512).astype(np.uint16)  # moderate magnitudes
    rows = len(pats)
    q = np.tile(np.arange(64, dtype=np.uint32) % 16, (rows, 1))
    w = pack(q, 4)
    s = pats.reshape(rows, 1)
    b = np.roll(pats, 5).reshape(rows, 1) ^ np.uint16(0x8000)
    got = oracle.bf16_to_f32(oracle.dequantize(w, s, b, 64, 4)).astype(np.float64)
    qs = q * oracle.bf16_to_f32(s).astype(np.float64)
    exact = qs + oracle.bf16_to_f32(b).astype(np.float64)
    bound = (np.abs(qs) + np.abs(exact)) * 2.0 ** -8
    assert np.all(np.abs(got - exact) <= bound * 1.0001 + 1e-38)
    # and the bound is tight enough to catch a dropped bias or scale
    assert not np.all(np.abs(qs - exact) <= bound)


# ---------------------------------------------------------------- quantize
# The requantize of absorbKVB (deepseekv3.go:662-669).  MLX's algorithm is not in
# the image and no reference fixture holds a quantized number, so the pins are
# what the algorithm fixes by construction: exact grids come back exactly (with
# the edge branch deciding the sign of the scale), the snap puts zero on the
# grid, constant groups reproduce, and the round-trip error of random data stays
# within a grid step.


def _grid(rng, rows, K, group, bits, base):
    """Rows whose every group is base + q * 2^-(bits) with q covering 0 .. 2^bits - 1
    at random positions: every value, product and sum is exact in bf16."""
    n = (1 << bits) - 1
    q = rng.integers(0, n + 1, size=(rows, K)).astype(np.uint32)
    for g in range(K // group):
        for r in range(rows):
            i, j = rng.choice(group, size=2, replace=False)
            q[r, g * group + i] = 0
            q[r, g * group + j] = n
    step = np.float32(2.0 ** -bits)
    w = np.float32(base) + q.astype(np.float32) * step
    w16 = oracle_f32_to_bf16(w)
    assert np.array_equal(oracle_bf16_to_f32(w16), w)
    return q, w16, step


def oracle_f32_to_bf16(f):
    from oracle import f32_to_bf16
    return f32_to_bf16(np.asarray(f, dtype=np.float32))


def oracle_bf16_to_f32(h):
    from oracle import bf16_to_f32
    return bf16_to_f32(h)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_quantize_exact_grid_min_edge(oracle, bits, group):
    """|min| > |max|: the edge is the minimum, the scale is +step, q is the grid."""
    rng = np.random.default_rng(bits * 7 + group)
    q, w, step = _grid(rng, 6, 256, group, bits, -0.5)
    wq, s, b = oracle.quantize(w, group, bits)
    assert np.array_equal(wq, pack(q, bits))
    assert np.all(s == oracle_f32_to_bf16(step)) and np.all(b == oracle_f32_to_bf16(-0.5))
    assert np.array_equal(oracle.dequantize(wq, s, b, group, bits), w)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_quantize_exact_grid_max_edge(oracle, bits, group):
    """|max| >= |min|: the edge is the maximum, the scale is -step and q counts down
    from it (q' = n - q), so the values still come back exactly."""
    rng = np.random.default_rng(bits * 11 + group)
    n = (1 << bits) - 1
    q, w, step = _grid(rng, 6, 256, group, bits, -0.25)
    wq, s, b = oracle.quantize(w, group, bits)
    assert np.array_equal(wq, pack(n - q, bits))
    assert np.all(s == oracle_f32_to_bf16(-step))
    assert np.all(b == oracle_f32_to_bf16(np.float32(-0.25) + n * step))
    assert np.array_equal(oracle.dequantize(wq, s, b, group, bits), w)


@pytest.mark.parametrize("bits,hi,scale,qmax", [(4, 0.9, 0.125, 15), (8, 0.99, 2.0 ** -7, 254)])
def test_quantize_snaps_zero_onto_the_grid(oracle, bits, hi, scale, qmax):
    """min -1, max just below 1: delta = range / n is off the powers of two, but
    q0 = rint(-1 / delta) is a power of two, so the snapped scale -1 / q0 is exact
    and the edge -1 and the zero element come back exactly.  Without the snap
    (scale = delta) zero would not.  The maximum: (0.8984375 + 1) * 8 = 15.19 -> 15;
    (0.98828125 + 1) * 128 = 254.5, a tie, -> 254 (rint rounds half to even)."""
    rng = np.random.default_rng(bits)
    K = 64
    n = (1 << bits) - 1
    v = rng.uniform(-0.9, 0.8, size=K).astype(np.float32)
    v[3], v[17], v[40] = -1.0, hi, 0.0
    w = oracle_f32_to_bf16(v).reshape(1, K)
    wq, s, b = oracle.quantize(w, 64, bits)
    assert oracle_bf16_to_f32(s)[0, 0] == np.float32(scale)
    assert oracle_bf16_to_f32(b)[0, 0] == np.float32(-1.0)
    got = oracle_bf16_to_f32(oracle.dequantize(wq, s, b, 64, bits))[0]
    assert got[3] == -1.0 and got[40] == 0.0
    assert unpack(wq, bits)[0, 17] == qmax
    # the unsnapped scale misses zero
    x = oracle_bf16_to_f32(w)[0]
    delta = np.float32((x.max() - x.min()) / np.float32(n))
    qz = np.rint(np.float32(1.0) / delta)
    assert qz * oracle_bf16_to_f32(oracle_f32_to_bf16(delta)) - 1.0 != 0.0


def test_quantize_constant_and_zero_groups(oracle):
    """A constant group has range 0: the scale is the 1e-7 floor with the max-edge
    sign, every q is 0 and the bias is the value itself.  A group of zeros, or of
    values below half the floor (1e-30 here), has q0 = 0: no snap, bias 0, and the
    group dequantizes to zeros."""
    K = 128
    w = oracle_f32_to_bf16(np.concatenate([np.full(32, 0.375), np.full(32, -2.5),
                                           np.zeros(32), np.full(32, 1e-30)]).astype(np.float32)
                           ).reshape(1, K)
    for bits in (4, 8):
        wq, s, b = oracle.quantize(w, 32, bits)
        assert np.all(wq == 0)
        sf, bf = oracle_bf16_to_f32(s)[0], oracle_bf16_to_f32(b)[0]
        assert bf.tolist() == [0.375, -2.5, 0.0, 0.0]
        assert sf[2] == sf[3] == oracle_bf16_to_f32(oracle_f32_to_bf16(np.float32(-1e-7)))
        assert np.all(sf < 0)
        want = w.copy()
        want[0, 96:] = 0
        assert np.array_equal(oracle.dequantize(wq, s, b, 32, bits), want)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_quantize_round_trip_error(oracle, bits, group):
    """Random data: every element comes back within one snapped grid step (the far
    end can sit up to one step past the last point before the clamp) plus the bf16
    roundings of scale, bias and the dequantized value; the mean error is a quarter
    step, as for rounding to a uniform grid, plus at 8 bits the bf16 roundings,
    which are then a sizeable part of a step (a q off by one would make it ~1)."""
    rng = np.random.default_rng(bits + group)
    n = (1 << bits) - 1
    w = oracle_f32_to_bf16(rng.standard_normal((40, 512)).astype(np.float32) *
                           np.float32(0.05))
    wq, s, b = oracle.quantize(w, group, bits)
    q = unpack(wq, bits)
    assert q.max() <= n
    x = oracle_bf16_to_f32(w).astype(np.float64)
    got = oracle_bf16_to_f32(oracle.dequantize(wq, s, b, group, bits)).astype(np.float64)
    sr = np.repeat(np.abs(oracle_bf16_to_f32(s)), group, axis=1).astype(np.float64)
    br = np.repeat(np.abs(oracle_bf16_to_f32(b)), group, axis=1).astype(np.float64)
    err = np.abs(got - x)
    assert np.all(err <= sr + 2.0 ** -8 * (n * sr + br + np.abs(x)))
    lo, hi = (0.2, 0.3) if bits == 4 else (0.25, 0.5)
    assert lo < np.mean(err / sr) < hi


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_quantize_matches_independent_numpy(oracle, bits, group):
    """The same steps vectorised in numpy float32 (grouping, branch selection and
    packing done independently): catches indexing and packing slips in the C
    loops."""
    rng = np.random.default_rng(3 * bits + group)
    n = np.float32((1 << bits) - 1)
    w = oracle_f32_to_bf16(rng.standard_normal((17, 384)).astype(np.float32))
    x = oracle_bf16_to_f32(w).reshape(17, -1, group)
    mn, mx = x.min(axis=-1, keepdims=True), x.max(axis=-1, keepdims=True)
    delta = (mx - mn) / n
    delta = np.where(delta > np.float32(1e-7), delta, np.float32(1e-7)).astype(np.float32)
    side = np.abs(mn) > np.abs(mx)
    scale = np.where(side, delta, -delta).astype(np.float32)
    edge = np.where(side, mn, mx).astype(np.float32)
    q0 = np.rint(edge / scale).astype(np.float32)
    snap = q0 != 0
    scale = np.where(snap, edge / np.where(snap, q0, np.float32(1)), scale).astype(np.float32)
    bias = np.where(snap, edge, np.float32(0)).astype(np.float32)
    q = np.clip(np.rint((x - bias) / scale), 0, n).astype(np.uint32).reshape(17, -1)
    wq, s, b = oracle.quantize(w, group, bits)
    assert np.array_equal(wq, pack(q, bits))
    assert np.array_equal(s, oracle_f32_to_bf16(scale[..., 0]))
    assert np.array_equal(b, oracle_f32_to_bf16(bias[..., 0]))


# ---------------------------------------------------------------- quantized_matmul

@pytest.mark.parametrize("bits", [4, 8])
def test_qmm_vs_fp64_and_numpy(oracle, bits):
    rng = np.random.default_rng(21 + bits)
    M, N, K = 3, 40, 256
    w, s, b = make_quant(rng, (N,), K, bits, 64)
    x = make_x(rng, M, K)
    y, yf = oracle.qmm(x, w, s, b, 64, bits, want_f32=True)
    y64 = oracle.qmm_f64(x, w, s, b, 64, bits)
    W = deq_numpy(w, s, b, bits, 64).astype(np.float64)
    ref = oracle.bf16_to_f32(x).astype(np.float64) @ W.T
    assert np.allclose(y64, ref, rtol=0, atol=1e-9)
    assert rel_err(yf, ref) < 1e-5
    assert np.array_equal(y, oracle.f32_to_bf16(yf))


def test_qmm_one_hot_selects_a_column(oracle):
    rng = np.random.default_rng(2)
    N, K = 16, 128
    w, s, b = make_quant(rng, (N,), K, 4, 64)
    W = oracle.dequantize(w, s, b, 64, 4)
    for k in (0, 5, 63, 64, 127):
        x = np.zeros((1, K), dtype=np.uint16)
        x[0, k] = 0x3F80  # 1.0
        y = oracle.qmm(x, w, s, b, 64, 4)
        assert np.array_equal(y[0], W[:, k])


def test_qmm_matches_torch_matmul(oracle):
    import torch

    rng = np.random.default_rng(8)
    M, N, K = 4, 64, 512
    w, s, b = make_quant(rng, (N,), K, 4, 64)
    x = make_x(rng, M, K)
    W = torch.from_numpy(oracle.bf16_to_f32(oracle.dequantize(w, s, b, 64, 4))).double()
    X = torch.from_numpy(oracle.bf16_to_f32(x)).double()
    ref = (X @ W.T).numpy()
    y = oracle.bf16_to_f32(oracle.qmm(x, w, s, b, 64, 4))
    assert rel_err(y, ref) < 4e-3


def test_qmm_linearity(oracle):
    rng = np.random.default_rng(13)
    N, K = 24, 256
    w, s, b = make_quant(rng, (N,), K, 8, 64)
    x1 = make_x(rng, 1, K)
    x2 = make_x(rng, 1, K)
    xs = oracle.f32_to_bf16(oracle.bf16_to_f32(x1) * 2)  # exact doubling
    _, y1 = oracle.qmm(x1, w, s, b, 64, 8, want_f32=True)
    _, y2 = oracle.qmm(xs, w, s, b, 64, 8, want_f32=True)
    assert np.array_equal(y2, y1 * 2)
    both = np.concatenate([x1, x2])
    _, yb = oracle.qmm(both, w, s, b, 64, 8, want_f32=True)
    _, y22 = oracle.qmm(x2, w, s, b, 64, 8, want_f32=True)
    assert np.array_equal(yb[0], y1[0]) and np.array_equal(yb[1], y22[0])


def test_cpu_fast_baseline_within_tolerance(oracle):
    rng = np.random.default_rng(17)
    for bits in (4, 8):
        w, s, b = make_quant(rng, (96,), 1024, bits, 64)
        x = make_x(rng, 5, 1024)
        ref = oracle.qmm_f64(x, w, s, b, 64, bits)
        fast = oracle.bf16_to_f32(oracle.qmm_cpu_fast(x, w, s, b, 64, bits))
        # the baseline uses the exact affine value s*q + b (no bf16 rounding of the
        # dequantized weight), so it sits a few 1e-3 away from the bf16-weight product
        assert rel_err(fast, ref) < 2e-2


def test_exact_mode_closed_forms(oracle):
    """DEQ_EXACT keeps s*q + b unrounded.  With s = 2^-4 and b = -0.5 every value
    (q - 8)/16 is a bf16, so all three definitions agree and one-hot x returns it;
    with s = 1 + 2^-7 the exact value 3.0390625 is not a bf16, and one-hot x
    returns it exactly, where the rounding modes return 3.03125 / 3.046875."""
    K = 64
    q = (np.arange(K, dtype=np.uint32) % 16).reshape(1, K)
    w = pack(q, 4)
    s = np.array([[0x3D80]], dtype=np.uint16)   # 2^-4
    b = np.array([[0xBF00]], dtype=np.uint16)   # -0.5
    want = (q[0].astype(np.float64) - 8.0) / 16.0
    for k in (0, 7, 8, 63):
        x = np.zeros((1, K), dtype=np.uint16)
        x[0, k] = 0x3F80
        for mode in (oracle.DEQ_MLX, oracle.DEQ_FUSED, oracle.DEQ_EXACT):
            assert oracle.qmm_f64(x, w, s, b, 64, 4, mode=mode)[0, 0] == want[k]
    w3 = pack(np.array([[3] + [0] * 63], dtype=np.uint32), 4)
    s3 = np.array([[0x3F81]], dtype=np.uint16)
    b3 = np.array([[0x3C80]], dtype=np.uint16)
    x = np.zeros((1, K), dtype=np.uint16)
    x[0, 0] = 0x3F80
    got = {m: oracle.qmm_f64(x, w3, s3, b3, 64, 4, mode=m)[0, 0]
           for m in (oracle.DEQ_MLX, oracle.DEQ_FUSED, oracle.DEQ_EXACT)}
    assert got[oracle.DEQ_EXACT] == 3.0390625
    assert got[oracle.DEQ_FUSED] == 3.03125 and got[oracle.DEQ_MLX] == 3.046875


def test_exact_mode_is_the_factored_sum(oracle):
    """EXACT equals s * sum(x q) + b * sum(x) per group in fp64 (the form the
    integer-domain kernels compute), far tighter than the bf16-weight modes do."""
    rng = np.random.default_rng(44)
    N, K = 24, 1024
    w, s, b = make_quant(rng, (N,), K, 4, 64)
    x = make_x(rng, 2, K)
    xf = oracle.bf16_to_f32(x).astype(np.float64).reshape(2, K // 64, 64)
    qf = unpack(w, 4).astype(np.float64).reshape(N, K // 64, 64)
    sf = oracle.bf16_to_f32(s).astype(np.float64)
    bf = oracle.bf16_to_f32(b).astype(np.float64)
    ref = (np.einsum("mgk,ngk->mng", xf, qf) * sf[None] + xf.sum(-1)[:, None, :] * bf[None]).sum(-1)
    ex = oracle.qmm_f64(x, w, s, b, 64, 4, mode=oracle.DEQ_EXACT)
    assert np.max(np.abs(ex - ref)) <= 1e-5 * np.max(np.abs(ref))
    mlx = oracle.qmm_f64(x, w, s, b, 64, 4, mode=oracle.DEQ_MLX)
    assert np.max(np.abs(mlx - ref)) > 100 * np.max(np.abs(ex - ref))


def _slip_cases(rng, N, K, G):
    """Planted kernel mistakes, each confined to one 64-value group of one row."""
    n, g = int(rng.integers(N)), int(rng.integers(1, G - 1))
    yield "dropped group", lambda s, b: (s.__setitem__((n, g), 0), b.__setitem__((n, g), 0))
    yield "neighbour's scale", lambda s, b: s.__setitem__((n, g), s[n, g + 1])
    yield "bias left out", lambda s, b: b.__setitem__((n, g), 0)


@pytest.mark.parametrize("K", [4096, 14336])
def test_parity_bound_accepts_kernels_and_catches_group_slips(oracle, K):
    """The per-element bound of the GPU tests (tests/parity.py) passes a result
    computed with either kernel definition, and fails every planted one-group slip."""
    import parity

    rng = np.random.default_rng(K)
    N, M = 48, 2
    w, s, b = make_quant(rng, (N,), K, 4, 64)
    x = make_x(rng, M, K)
    ref = parity.DenseRef(x, w, s, b, 64, 4)
    for mode in (oracle.DEQ_EXACT, oracle.DEQ_FUSED):
        good = oracle.qmm(x, w, s, b, 64, 4, mode=mode)
        parity.check_dense(good, ref, what=f"mode {mode}")
    for name, plant in _slip_cases(rng, N, K, K // 64):
        s2, b2 = s.copy(), b.copy()
        plant(s2, b2)
        bad = oracle.qmm(x, w, s2, b2, 64, 4, mode=oracle.DEQ_EXACT)
        with pytest.raises(AssertionError, match="per-element"):
            parity.check_dense(bad, ref, what=name)


def test_max_abs_rel_metric_misses_a_typical_group_drop(oracle):
    """Why the per-element bound exists: on 14336-deep rows, dropping the group of
    median contribution in one row stays inside max-abs-rel 2e-2 but fails the
    bound by a wide margin."""
    import parity

    rng = np.random.default_rng(3)
    N, M, K = 512, 2, 14336
    w, s, b = make_quant(rng, (N,), K, 4, 64)
    x = make_x(rng, M, K)
    ref = parity.DenseRef(x, w, s, b, 64, 4)
    n = 7
    contrib = []
    for g in range(K // 64):  # row n's per-group contribution to y[0, n]
        s1, b1 = s.copy(), b.copy()
        s1[n, g] = b1[n, g] = 0
        contrib.append(ref.exact[0, n] - oracle.qmm_f64(x[:1], w[n:n + 1], s1[n:n + 1],
                                                         b1[n:n + 1], 64, 4,
                                                         mode=oracle.DEQ_EXACT)[0, 0])
    g = int(np.argsort(np.abs(contrib))[len(contrib) // 2])
    s2, b2 = s.copy(), b.copy()
    s2[n, g] = b2[n, g] = 0
    bad = oracle.qmm(x, w, s2, b2, 64, 4, mode=oracle.DEQ_EXACT)
    assert rel_err(oracle.bf16_to_f32(bad), ref.mlx) <= 2e-2
    with pytest.raises(AssertionError, match="per-element"):
        parity.check_dense(bad, ref)


def test_switch_bound_catches_a_down_group_slip(oracle):
    """SwitchGLU outputs at configuration 3's expert shape (2048 -> 512 -> 2048):
    both kernel definitions pass the per-slot bound, and so does the MLX-definition
    output, whose intermediates flip far more often than a kernel's.  Dropping the
    down group of median contribution from one row fails the bound."""
    import parity

    rng = np.random.default_rng(46)
    T, k, E, D, I = 3, 2, 8, 2048, 512
    gate = make_quant(rng, (E, I), D, 4, 64)
    up = make_quant(rng, (E, I), D, 4, 64)
    down = make_quant(rng, (E, D), I, 4, 64)
    x = make_x(rng, T, D)
    inds = np.array([[5, 1], [6, 2], [4, 7]], dtype=np.int32)
    sref = parity.SwitchRef(x, inds, gate, up, down)
    for mode in (oracle.DEQ_EXACT, oracle.DEQ_FUSED, oracle.DEQ_MLX):
        got = oracle.switch_glu(x, inds, gate, up, down, mode=mode)
        parity.check_switch(got, sref, what=f"mode {mode}")
    e, n = 5, 11  # token 0's first expert, output row 11
    base = parity.f64(oracle.switch_glu(x, inds, gate, up, down, mode=oracle.DEQ_EXACT,
                                        token_sel=np.array([0])))[0, 0, n]

    def dropped(g):
        sd, bd = down[1].copy(), down[2].copy()
        sd[e, n, g] = bd[e, n, g] = 0
        return oracle.switch_glu(x, inds, gate, up, (down[0], sd, bd), mode=oracle.DEQ_EXACT)

    contrib = [abs(parity.f64(dropped(g))[0, 0, n] - base) for g in range(I // 64)]
    g = int(np.argsort(contrib)[len(contrib) // 2])
    with pytest.raises(AssertionError, match="per-element"):
        parity.check_switch(dropped(g), sref)


# ---------------------------------------------------------------- gather / SwitchGLU

def test_gather_single_expert_reduces_to_qmm(oracle):
    rng = np.random.default_rng(31)
    N, K = 32, 128
    w, s, b = make_quant(rng, (1, N), K, 4, 64)
    x = make_x(rng, 5, K)
    g = oracle.gather_qmm(x, w, s, b, np.arange(5), np.zeros(5, dtype=np.int32))
    q = oracle.qmm(x, w[0], s[0], b[0])
    assert np.array_equal(g, q)


def test_gather_picks_expert_slices(oracle):
    rng = np.random.default_rng(32)
    E, N, K = 5, 16, 128
    w, s, b = make_quant(rng, (E, N), K, 4, 64)
    x = make_x(rng, 3, K)
    xrow = np.array([2, 0, 1, 2])
    ex = np.array([4, 1, 1, 0])
    g = oracle.gather_qmm(x, w, s, b, xrow, ex)
    for i in range(4):
        q = oracle.qmm(np.ascontiguousarray(x[xrow[i]:xrow[i] + 1]), w[ex[i]], s[ex[i]], b[ex[i]])
        assert np.array_equal(g[i], q[0])
    with pytest.raises(ValueError):
        oracle.gather_qmm(x, w, s, b, xrow, np.array([0, 1, 5, 0]))


def test_switch_glu_is_the_op_chain(oracle):
    """switch_glu == gather(down, bf16(silu(gate)) * up) with each op rounded."""
    rng = np.random.default_rng(41)
    T, k, E, D, I = 3, 2, 4, 128, 64
    gate = make_quant(rng, (E, I), D, 4, 64)
    up = make_quant(rng, (E, I), D, 4, 64)
    down = make_quant(rng, (E, D), I, 4, 64)
    x = make_x(rng, T, D)
    inds = np.array([[0, 3], [2, 2 - 1], [3, 0]], dtype=np.int32)
    out = oracle.switch_glu(x, inds, gate, up, down)
    xr = np.repeat(np.arange(T), k)
    ex = inds.reshape(-1)
    g = oracle.bf16_to_f32(oracle.gather_qmm(x, *gate, xr, ex))
    u = oracle.bf16_to_f32(oracle.gather_qmm(x, *up, xr, ex))
    r = lambda v: oracle.bf16_to_f32(oracle.f32_to_bf16(v.astype(np.float32)))
    sig = r(1.0 / (1.0 + np.exp(-g.astype(np.float64))))
    h = oracle.f32_to_bf16(r(g * sig) * u)
    d = oracle.gather_qmm(h, *down, np.arange(T * k), ex)
    assert rel_err(oracle.bf16_to_f32(out.reshape(T * k, D)), oracle.bf16_to_f32(d)) < 1e-2
    sel = oracle.switch_glu(x, inds, gate, up, down, token_sel=np.array([2]))
    assert np.array_equal(sel[0], out[2])


# ---------------------------------------------------------------- reference fixture

def test_tensor_bytes_formula_matches_reference_fixture():
    """The algorithmic byte count used for the roofline equals the reference's
    TensorQuantizedBytes (quant/oq.go:315-332) on its own fixture rows."""
    from fastmlx_amd.roofline import quantized_tensor_bytes

    with open(os.path.join(GOLDEN, "oq_tensor_bytes.json")) as f:
        rows = json.load(f)["tensor_bytes"]
    assert rows
    for r in rows:
        assert quantized_tensor_bytes(r["shape"], r["bits"], r["gs"], r["mode"]) == r["bytes"], r


# ---- MoE routers -------------------------------------------------------------

def _routing_fixture():
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                        "deepseek_routing.json")
    with open(path) as f:
        return json.load(f)["routing"]


@pytest.mark.parametrize("case", _routing_fixture(), ids=lambda c: c["label"])
def test_route_group_oracle_matches_reference_fixture(oracle, case):
    """The reference's own vectors for GroupExpertSelect, compared the way
    TestDeepseekV3GroupExpertSelectParity does (compute/models/deepseekv3_test.go:
    130-163): the expert -> weight map at 1e-5 relative."""
    inds, sc = oracle.route_group_topk(case["gates"], case["bias"], case["top_k"],
                                       case["n_group"], case["topk_group"],
                                       case["routed_scaling_factor"], case["norm_topk_prob"])
    got = dict(zip(inds[0].tolist(), sc[0].tolist()))
    want = dict(zip(case["inds"], case["scores"]))
    assert set(got) == set(want)
    for e, w in want.items():
        assert abs(got[e] - w) <= 1e-5 * abs(w)


def test_route_group_oracle_invariants(oracle):
    rng = np.random.default_rng(71)
    T, E, k = 40, 64, 6
    gates = rng.standard_normal((T, E)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
    # keeping every group is the same as one group
    a = oracle.route_group_topk(gates, bias, k, 8, 8, 1.7, True)
    b = oracle.route_group_topk(gates, bias, k, 1, 1, 1.7, True)
    assert np.array_equal(a[0], b[0]) and np.allclose(a[1], b[1])
    # weights are the unbiased sigmoids of the picks, renormalized and scaled
    sig = 1.0 / (1.0 + np.exp(-gates.astype(np.float64)))
    inds, sc = oracle.route_group_topk(gates, bias, k, 8, 3, 2.5, True)
    picked = np.take_along_axis(sig, inds.astype(np.int64), axis=1)
    assert np.allclose(sc, 2.5 * picked / picked.sum(axis=1, keepdims=True))
    # without bias every score is positive, so every pick lies in a kept group:
    # at most topk_group distinct groups
    inds, _ = oracle.route_group_topk(gates, None, k, 8, 3, 1.0, False)
    assert all(len(set((r // 8).tolist())) <= 3 for r in inds)
    # the kept groups are the ones with the best two-expert sums
    g2 = np.sort(sig.reshape(T, 8, 8), axis=2)[:, :, -2:].sum(axis=2)
    best = np.argsort(-g2, axis=1, kind="stable")[:, :3]
    for t in range(T):
        assert set((inds[t] // 8).tolist()) <= set(best[t].tolist())
    # picks come out in descending biased score
    ninds, _ = oracle.route_group_topk(gates, bias, E, 1, 1, 1.0, False)
    biased = sig + bias
    assert np.all(np.diff(np.take_along_axis(biased, ninds.astype(np.int64), 1), axis=1) <= 0)


def test_route_softmax_oracle_closed_forms(oracle):
    rng = np.random.default_rng(72)
    T, E, k = 30, 128, 10
    x = rng.standard_normal((T, E)).astype(np.float32)
    inds, w = oracle.route_softmax_topk(x, k, norm=True)
    # the renormalized top-k of a softmax is the softmax of the top-k logits
    sel = np.take_along_axis(x.astype(np.float64), inds.astype(np.int64), axis=1)
    ref = np.exp(sel - sel.max(axis=1, keepdims=True))
    assert np.allclose(w, ref / ref.sum(axis=1, keepdims=True), rtol=1e-12)
    # the picks are the k largest logits, in descending order
    assert np.array_equal(inds, np.argsort(-x, axis=1, kind="stable")[:, :k])
    # with every expert and no renormalization the weights are the softmax
    _, full = oracle.route_softmax_topk(x, E, norm=False)
    assert np.allclose(full.sum(axis=1), 1.0)
    # equal gates go to the lower index
    tied = np.zeros((1, 16), np.float32)
    tied[0, [3, 9, 12]] = 2.0
    ti, _ = oracle.route_softmax_topk(tied, 4, norm=True)
    assert ti[0].tolist() == [3, 9, 12, 0]
