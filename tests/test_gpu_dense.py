"""GPU parity: dequantize (bit-exact) and quantized_matmul vs the oracle.

Inputs are seeded numpy tensors shared byte-for-byte by the HIP path and the
CPU oracle.  Every product is held to two bars:
- the north-star metric, max|y - y_ref| / max|y_ref| <= 2e-2 on bf16 outputs
  against the fp32 oracle with the MLX dequant;
- the per-element fp64 bound of tests/parity.py, which a slip in one 64-value
  group of one row fails.
"""
import numpy as np
import pytest
import torch

from gpu_util import announce, to_dev, to_np
from synth import make_quant, make_x, rel_err

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_dequantize_bit_exact(gpu, oracle, bits, group):
    rng = np.random.default_rng(100 + bits * 10 + group)
    N, K = 96, 512
    w, s, b = make_quant(rng, (N,), K, bits, group)
    announce(f"dequantize bits={bits} group={group} N={N} K={K}")
    from fastmlx_amd import ops

    out = ops.dequantize(to_dev(w, gpu), to_dev(s, gpu), to_dev(b, gpu), group, bits)
    torch.cuda.synchronize()
    got = to_np(out)
    ref = oracle.dequantize(w, s, b, group, bits)
    assert got.shape == ref.shape
    assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} mismatching elements"


@pytest.mark.parametrize("bits", [4, 8])
def test_dequantize_exhaustive_q_and_bf16_sweep(gpu, oracle, bits):
    """Every q value against a sweep of bf16 scale/bias bit patterns (incl. subnormal,
    negative, large and tie-producing values): bit-exact with the oracle."""
    rng = np.random.default_rng(7 + bits)
    group = 64
    nq = 1 << bits
    # bf16 patterns: random over all finite exponents plus specials
    pats = rng.integers(0, 0x7F80, size=2048, dtype=np.uint32).astype(np.uint16)
    pats = np.concatenate([pats, pats | 0x8000,
                           np.array([0x0000, 0x8000, 0x0001, 0x007F, 0x3F80, 0xBF80, 0x4300,
                                     0x3C00, 0x7F7F, 0xFF7F], dtype=np.uint16)])
    rows = len(pats)
    K = group * 4  # four groups per row
    q = np.tile(np.arange(K, dtype=np.uint32) % nq, (rows, 1))
    from synth import pack

    w = pack(q, bits)
    s = np.stack([pats, np.roll(pats, 1), np.roll(pats, 7), pats[::-1]], axis=1).astype(np.uint16)
    bb = np.stack([np.roll(pats, 3), pats, pats[::-1], np.roll(pats, 11)], axis=1).astype(np.uint16)
    s = np.ascontiguousarray(s)
    bb = np.ascontiguousarray(bb)
    announce(f"dequantize sweep bits={bits} rows={rows}")
    from fastmlx_amd import ops

    out = ops.dequantize(to_dev(w, gpu), to_dev(s, gpu), to_dev(bb, gpu), group, bits)
    torch.cuda.synchronize()
    got = to_np(out)
    ref = oracle.dequantize(w, s, bb, group, bits)
    nan_ref = (ref & 0x7FFF) > 0x7F80
    assert np.array_equal(got[~nan_ref], ref[~nan_ref])
    assert np.all((got[nan_ref] & 0x7FFF) > 0x7F80)


def _qmm_case(gpu, oracle, M, N, K, bits, group, seed, rows_checked=None, bias=False):
    """One quantized_matmul through the C ABI, checked on the selected rows of x
    (all rows by default) element by element against the fp64 oracle
    (tests/parity.py) and by the 2e-2 max-abs-rel metric."""
    import parity

    rng = np.random.default_rng(seed)
    w, s, b = make_quant(rng, (N,), K, bits, group)
    x = make_x(rng, M, K)
    bvec = make_x(rng, N) if bias else None
    announce(f"quantized_matmul M={M} N={N} K={K} bits={bits} group={group} bias={bias}")
    from fastmlx_amd import ops

    y = ops.quantized_matmul(to_dev(x, gpu), to_dev(w, gpu), to_dev(s, gpu), to_dev(b, gpu),
                             True, group, bits, bias=None if bvec is None else to_dev(bvec, gpu))
    torch.cuda.synchronize()
    got = to_np(y)
    sel = np.arange(M) if rows_checked is None else rows_checked
    ref = parity.DenseRef(np.ascontiguousarray(x[sel]), w, s, b, group, bits)
    worst = parity.check_dense(got[sel], ref, bias16=bvec,
                               what=f"M={M} N={N} K={K} bits={bits} group={group}")
    e = rel_err(oracle.bf16_to_f32(got[sel]), ref.mlx if bvec is None else
                oracle.bf16_to_f32(oracle.f32_to_bf16(ref.mlx + oracle.bf16_to_f32(bvec)[None])))
    print(f"  max-abs-rel {e:.3e}; per-element bound used up to {worst:.2f}")
    return e


@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("bits", [4, 8])
def test_qmv_config0_shape(gpu, oracle, M, bits):
    # config 0: 2048x2048, group 64
    # the decode GEMV works on the exact affine value s*q + b (no bf16 rounding of
    # the dequantized weight) and sums in another order; it must still meet 2e-2
    _qmm_case(gpu, oracle, M, 2048, 2048, bits, 64, seed=1000 + M + bits)


@pytest.mark.parametrize("M", [2, 3, 4])
@pytest.mark.parametrize("N", [1024, 4096])
def test_qmv_long_rows_small_m(gpu, oracle, M, N):
    """int4 at M = 2-4 on 14336-deep rows: the register GEMV's shapes for narrow
    (<= 2048) and wide outputs."""
    _qmm_case(gpu, oracle, M, N, 14336, 4, 64, seed=1100 + M + N)


@pytest.mark.parametrize("group", [32, 128])
def test_qmv_other_groups(gpu, oracle, group):
    _qmm_case(gpu, oracle, 1, 384, 1024, 4, group, seed=31 + group)
    _qmm_case(gpu, oracle, 7, 384, 1024, 8, group, seed=37 + group)


@pytest.mark.parametrize("M", [5, 6, 7, 8, 16, 32, 64, 100, 128, 300])
@pytest.mark.parametrize("bits", [4, 8])
def test_qmm_mfma_shapes(gpu, oracle, M, bits):
    _qmm_case(gpu, oracle, M, 1024 + 64, 2048, bits, 64, seed=2000 + M + bits)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("N,K", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336), (1024, 16384)])
def test_int8_small_m_shapes(gpu, oracle, M, N, K):
    """int8 at 1 <= M <= 8: the register GEMV (at M >= 5 only M of its 8 x-row
    slots built) on the narrower outputs and at M = 1 (rows of 14336 and 16384
    values in its eight-slice, two-chunk form), and the dequantizing skinny walk on
    long rows from M = 2, on 14336 outputs from M = 3 and on 4096 outputs at M = 8."""
    _qmm_case(gpu, oracle, M, N, K, 8, 64, seed=14000 + M + N // 1024)


@pytest.mark.parametrize("M,N,K,bits,group", [(6, 1024, 14336, 4, 64), (7, 1000, 8192, 4, 64),
                                               (5, 2048, 9216, 8, 32), (6, 3000, 4096, 8, 64)])
def test_register_gemv_partial_rows(gpu, oracle, M, N, K, bits, group):
    """The register GEMV with 5..7 of its 8 x-row slots built, on the 8-slice form
    of long rows and on ragged row counts (int8 long rows in group 32, which the
    int8 skinny walk does not take)."""
    _qmm_case(gpu, oracle, M, N, K, bits, group, seed=15000 + M * 7 + N + K + bits)


def test_qmm_ragged_n(gpu, oracle):
    # N not a multiple of any tile, K a multiple of 32 only
    _qmm_case(gpu, oracle, 1, 333, 96, 4, 32, seed=5)
    _qmm_case(gpu, oracle, 37, 333, 96, 4, 32, seed=6)
    _qmm_case(gpu, oracle, 130, 77, 160, 8, 32, seed=7)


@pytest.mark.parametrize("M,N,K,bits,group", [
    (65, 333, 64, 4, 64),        # one K step; 128x256 tile with ragged N
    (129, 1000, 320, 4, 32),     # five steps (tail only); first 256x128 size
    (257, 256, 448, 4, 64),      # seven steps: one six-step pass plus a tail of one
    (200, 192, 640, 4, 128),     # ten steps: a tail of four
    (300, 520, 832, 8, 64),      # thirteen steps, 8-bit, ragged M and N
    (100, 384, 1024, 8, 32),     # 8-bit at M <= 128 takes the 256x128 tile
    (512, 128, 2048, 8, 128),
    (1000, 2048, 768, 4, 64),
    (33, 1000, 1024, 4, 64),     # the smallest M on this kernel
    (64, 520, 3072, 8, 128),
])
def test_qmm_prefill_tiles(gpu, oracle, M, N, K, bits, group):
    """The M > 32 prefill GEMM: every step-count remainder of its six-step loop,
    both tiles, ragged M and N, both bit widths and every group size."""
    _qmm_case(gpu, oracle, M, N, K, bits, group, seed=7000 + M + N + K + bits + group)


@pytest.mark.parametrize("M,N,K,bits,group,bias", [
    (300, 512, 2048, 4, 64, True),     # 8 tiles -> 4 K parts each (fixup adds the bias)
    (130, 700, 4096, 8, 32, False),    # 8-bit, group 32, ragged M and N, parts only
    (1000, 2048, 8192, 4, 128, False), # 64 tiles x 4 parts
    (512, 16640, 1024, 4, 32, True),   # 260 tiles: 256 whole, the last 4 in 2 parts each
                                       # (group 32 keeps M = 512 off the wide GEMM)
])
def test_qmm_prefill_k_split(gpu, oracle, M, N, K, bits, group, bias):
    """Prefill tiles of a part-full last wave are computed in K parts summed by a
    fixup kernel; whole and split tiles must both match the oracle, twice in a row
    (the partial workspace is overwritten, never accumulated)."""
    rows = None if M <= 130 else np.unique(np.concatenate([[0, M - 1], np.arange(0, M, 37)]))
    e1 = _qmm_case(gpu, oracle, M, N, K, bits, group, seed=8800 + M + K + bits, rows_checked=rows,
                   bias=bias)
    e2 = _qmm_case(gpu, oracle, M, N, K, bits, group, seed=8800 + M + K + bits, rows_checked=rows,
                   bias=bias)
    assert e1 == e2


@pytest.mark.parametrize("M", [5, 7, 8, 9, 13, 16, 17, 24, 25, 31, 32])
@pytest.mark.parametrize("bits,group,K", [(4, 64, 192), (4, 128, 1024), (8, 32, 96),
                                          (8, 64, 2048)])
def test_skinny_mfma_rows_and_groups(gpu, oracle, M, bits, group, K):
    """The 5 <= M <= 32 MFMA GEMV: every count of live accumulator rows, ragged N,
    both bit widths and the group sizes it accepts."""
    _qmm_case(gpu, oracle, M, 333, K, bits, group, seed=900 + M * 3 + bits + group)


@pytest.mark.parametrize("M", [3, 4, 5, 8, 9, 16, 17, 32])
@pytest.mark.parametrize("N,K", [
    (8200, 1024),   # 32-row blocks (N >= 8192), ragged N, one 4-unit step per wave
    (2100, 8192),   # 16-row blocks with 8-unit steps, ragged N
    (2064, 256),    # a single step: three of the four waves of a block get none
    (2048, 768),    # three steps over four waves
    (4096, 4352),   # seventeen steps: uneven slices and an odd step count per wave
])
def test_qmvs_blocks_and_steps(gpu, oracle, M, N, K):
    """The int4 group-64 skinny GEMV (qmvs): both block heights, both step sizes,
    slices with no steps or an odd number of them, one and two 16-row x tiles;
    M = 3 and 4 take it on 4096 or more outputs (the dot2 GEMV below that)."""
    _qmm_case(gpu, oracle, M, N, K, 4, 64, seed=9100 + M * 7 + N + K)


@pytest.mark.parametrize("N,K,bias", [
    (1001, 8192, False),   # four 2048-deep slices, rows not a multiple of the 8-row wave
    (77, 16384, True),     # eight slices (the largest block), bias epilogue
    (77, 32768, False),    # sixteen slices: not taken by the slice kernel
    (264, 14336, False),   # the down-projection depth (16-row waves)
    (16392, 14336, True),  # past 16384 outputs: 8-row waves, ragged, bias epilogue
    (2056, 4096, True),    # two slices x two 8-row groups per block, ragged
    (1001, 4096, False),   # two slices x two 2-row groups per block
    (28680, 4096, False),  # two slices on a tall matrix (rows past 16384), ragged
    (8196, 4096, True),    # two slices of 4-row waves (8192 to 32767 outputs), ragged
    (32776, 4096, False),  # two slices of 8-row waves again past 32767 outputs
    (2050, 2048, True),    # one slice (2048-deep rows), ragged rows, bias epilogue
    (77, 2048, False),     # one slice, fewer rows than one block's eight
    (520, 6144, False),    # three slices: not taken by the slice kernel
])
def test_qmv1_slice_shapes(gpu, oracle, N, K, bias):
    """M = 1 GEMV over 2048-deep K slices (qmv1_slice_kernel) and its neighbours."""
    _qmm_case(gpu, oracle, 1, N, K, 4, 64, seed=9300 + N + K, bias=bias)


@pytest.mark.parametrize("M", [9, 17, 33, 48, 64])
@pytest.mark.parametrize("N,K,bias", [
    (8200, 1024, False),  # wide: 32-row W tiles, 4 up-front parts of one step (64-row x: 2 pipelined)
    (4100, 2048, True),   # 4 parts of two steps, ragged last row block, bias in the fixup
    (1022, 4096, False),  # narrow: 8 up-front parts of two steps; N % 4 != 0 (scalar fixup)
    (2050, 8192, False),  # long rows: 8 pipelined parts of four steps, N % 4 != 0
    (4096, 7936, False),  # 31 steps: too many for the up-front walk, which falls back
    (130, 256, True),     # one step: a single part stores bf16 directly
])
def test_qmvw_parts_and_walks(gpu, oracle, M, N, K, bias):
    """The int4 group-64 product with x shared through LDS (qmvw, 9 <= M <= 64 on
    wide or long shapes, every shape from M = 17): each plan branch (pipelined and
    up-front walks, one or several K parts, 16- and 32-row W tiles, 16 to 64 x
    rows), ragged rows, both fixup forms and the bias epilogue.  Two calls in a
    row agree exactly (the parts are summed in a fixed order)."""
    rows = np.unique(np.array([0, 1, M // 2, M - 2, M - 1]))
    y1 = _qmm_case(gpu, oracle, M, N, K, 4, 64, seed=9400 + M * 5 + N + K, rows_checked=rows,
                   bias=bias)
    del y1
    from fastmlx_amd import ops

    rng = np.random.default_rng(1)
    w, s, b = make_quant(rng, (N,), K, 4, 64)
    x = make_x(rng, M, K)
    dx, dw, ds, db = (to_dev(t, gpu) for t in (x, w, s, b))
    r1 = to_np(ops.quantized_matmul(dx, dw, ds, db, True, 64, 4))
    r2 = to_np(ops.quantized_matmul(dx, dw, ds, db, True, 64, 4))
    torch.cuda.synchronize()
    assert np.array_equal(r1, r2)


@pytest.mark.parametrize("M", [9, 16, 17, 32, 33, 64])
@pytest.mark.parametrize("N,K,bias", [
    (8200, 1024, False),  # wide: parts of one step, ragged N
    (4100, 2048, True),   # 4 parts of two steps, ragged last row block, bias in the fixup
    (2050, 8192, False),  # long rows: 8 parts of four steps, N % 4 != 0 (scalar fixup)
    (4096, 7936, False),  # 31 steps: uneven parts, an odd step count
    (130, 256, True),     # one step: a single part stores bf16 directly
])
def test_qmvw_int8(gpu, oracle, M, N, K, bias):
    """The int8 group-64 skinny walk (qmvw with BITS = 8, weights dequantized to
    bf16 in 256-byte row slices per step), on every x-tile count and part plan it
    takes, including shapes whose M <= 16 rows stay off it; two calls in a row
    agree exactly."""
    rows = np.unique(np.array([0, 1, M // 2, M - 2, M - 1]))
    _qmm_case(gpu, oracle, M, N, K, 8, 64, seed=9600 + M * 5 + N + K, rows_checked=rows,
              bias=bias)
    from fastmlx_amd import ops

    rng = np.random.default_rng(2)
    w, s, b = make_quant(rng, (N,), K, 8, 64)
    x = make_x(rng, M, K)
    dx, dw, ds, db = (to_dev(t, gpu) for t in (x, w, s, b))
    r1 = to_np(ops.quantized_matmul(dx, dw, ds, db, True, 64, 8))
    r2 = to_np(ops.quantized_matmul(dx, dw, ds, db, True, 64, 8))
    torch.cuda.synchronize()
    assert np.array_equal(r1, r2)


@pytest.mark.parametrize("M,N,K,bits,group", [
    (384, 1024, 1024, 4, 64),    # the threshold M
    (383, 1024, 1024, 4, 64),    # one row below it: the prefill GEMM
    (128, 8192, 4096, 4, 64),    # outputs twice the depth: the wide GEMM from M = 128
    (127, 8192, 4096, 8, 64),    # one row below: the prefill GEMM
    (512, 14336, 4096, 8, 64),   # 224 tiles on 256 CUs: one whole tile per block
    (768, 1024, 1024, 4, 64),
    (1024, 1024, 1024, 4, 64),
    (1500, 4104, 2048, 4, 32),   # group 32: the prefill GEMM's 64-row tile instead
    (1024, 2048, 4096, 4, 128),  # group 128: likewise
    (1100, 1032, 3072, 8, 64),   # ragged M, N not a multiple of the 256-output tile
    (2048, 4096, 1024, 8, 32),
    (1000, 4096, 14336, 4, 64),  # 128-row tiles, stream-K pieces of 112 steps
    (2048, 4096, 14336, 8, 64),  # 256-row tiles, two pieces per tile
    (1300, 14336, 4096, 4, 64),  # whole tiles, then stream-K pieces of uneven length
])
def test_wide_gemm_shapes(gpu, oracle, M, N, K, bits, group):
    """Prefill-sized products (M >= 384, or M >= 128 where N >= 2K): the
    hand-written wide MFMA GEMM (group 64, K a multiple of 256) with its stream-K
    split of the K range or one whole tile per block, or the prefill GEMM for the
    other group sizes and just below the thresholds; per-element bound against the
    fp64 oracle."""
    rows = np.unique(np.array([0, 1, M // 3, M // 2, M - 2, M - 1]))
    _qmm_case(gpu, oracle, M, N, K, bits, group, seed=9700 + M + N + K + bits + group,
              rows_checked=rows)


@pytest.mark.parametrize("M,N,K,bits", [(1000, 4096, 14336, 4), (2048, 4096, 14336, 8),
                                        (2048, 14336, 4096, 4)])
def test_wide_gemm_repeated_calls(gpu, M, N, K, bits):
    """Six calls in a row on every row and output, against a torch fp32 product of
    the dequantized weights (fmxq dequantize is bit-exact against the oracle).  A
    slip in the pipelined waits shows up as a 32-row slab of one step's x read
    stale in some calls only, so one call is not enough.  Gross-error bound:
    2e-2 of the rms output plus 1e-2 of the element (bf16 output rounding and fp32
    order differences stay 5x below it; a stale 64-deep step of x is far above)."""
    from fastmlx_amd import ops

    announce(f"wide GEMM repeated calls M={M} N={N} K={K} bits={bits}")
    rng = np.random.default_rng(M + N + bits)
    w, s, b = make_quant(rng, (N,), K, bits, 64)
    x = make_x(rng, M, K)
    dx, dw, ds, db = (to_dev(t, gpu) for t in (x, w, s, b))
    wd = ops.dequantize(dw, ds, db, 64, bits).view(torch.bfloat16).float()
    ref = dx.view(torch.bfloat16).float() @ wd.t()
    rms = float(ref.pow(2).mean().sqrt())
    bound = 0.02 * rms + 0.01 * ref.abs()
    for call in range(6):
        y = ops.quantized_matmul(dx, dw, ds, db, True, 64, bits).view(torch.bfloat16).float()
        bad = int(((y - ref).abs() > bound).sum())
        assert bad == 0, f"call {call}: {bad} of {y.numel()} outputs off the fp32 product"


def test_qmvs_bias(gpu, oracle):
    _qmm_case(gpu, oracle, 12, 8256, 512, 4, 64, seed=9201, bias=True)
    _qmm_case(gpu, oracle, 30, 2080, 1024, 4, 64, seed=9202, bias=True)


@pytest.mark.parametrize("M", [1, 9, 70, 300])
def test_qlinear_bias_epilogue(gpu, oracle, M):
    _qmm_case(gpu, oracle, M, 512, 1024, 4, 64, seed=300 + M, bias=True)


@pytest.mark.parametrize("N,K", [(14336, 4096), (4096, 14336)])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [1, 5, 64, 512, 2048])
def test_config2_full_shapes(gpu, oracle, N, K, bits, M):
    """Config 2 (verify/prefill) at full size; the oracle evaluates a sample of rows."""
    rows = None if M <= 8 else np.random.default_rng(M).choice(M, size=6, replace=False)
    if rows is not None:
        rows = np.sort(np.append(rows, [0, M - 1]))
    _qmm_case(gpu, oracle, M, N, K, bits, 64, seed=4000 + M + bits + K, rows_checked=rows)


# The Llama-3-8B projections of BASELINE config 1 (llama.go:403-428): q/o 4096x4096,
# k/v 1024x4096 (GQA, 8 kv heads), gate/up 14336x4096, down 4096x14336.
LLAMA_SHAPES = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]


@pytest.mark.parametrize("M", [1, 2, 4, 8, 16, 32])
@pytest.mark.parametrize("N,K", LLAMA_SHAPES)
def test_config1_stack_shapes(gpu, oracle, M, N, K):
    """Config 1 at every batch the bench times, through the same dispatch
    (quantized_matmul picks the M=1 slice GEMV, the M <= 8 register GEMV or the
    skinny MFMA walk by M and shape); up to 8 rows of x are checked per case."""
    rows = None if M <= 8 else np.unique(np.concatenate(
        [[0, M - 1], np.random.default_rng(M).choice(M, size=4, replace=False)]))
    _qmm_case(gpu, oracle, M, N, K, 4, 64, seed=12000 + M * 31 + N // 1024 + K // 1024,
              rows_checked=rows)


@pytest.mark.parametrize("M", [1, 32])
def test_tied_head_vocab(gpu, oracle, M):
    """The tied lm_head (llama.go:433-437) is qlinear on the embedding triple at
    vocab x hidden = 128256 x 4096: the largest single decode product."""
    rows = None if M == 1 else np.array([0, 13, M - 1])
    _qmm_case(gpu, oracle, M, 128256, 4096, 4, 64, seed=13000 + M, rows_checked=rows)


@pytest.mark.parametrize("M,N,K", [(5, 1024, 4096), (16, 1024, 4096), (32, 512, 14336),
                                   (64, 4096, 2048), (200, 256, 4096)])
def test_split_k_shapes_repeat(gpu, oracle, M, N, K):
    """Shapes with few output tiles take the split-K path; the per-stream workspace
    must come back to zero after every call, so two calls in a row agree exactly."""
    from fastmlx_amd import ops

    rng = np.random.default_rng(M * 7 + N)
    w, s, b = make_quant(rng, (N,), K, 4, 64)
    x = make_x(rng, M, K)
    dx, dw, ds, db = (to_dev(t, gpu) for t in (x, w, s, b))
    announce(f"split-K M={M} N={N} K={K}")
    y1 = to_np(ops.quantized_matmul(dx, dw, ds, db, True, 64, 4))
    y2 = to_np(ops.quantized_matmul(dx, dw, ds, db, True, 64, 4))
    torch.cuda.synchronize()
    rows = np.unique(np.array([0, M // 2, M - 1]))
    import parity

    parity.check_dense(y1[rows], parity.DenseRef(np.ascontiguousarray(x[rows]), w, s, b, 64, 4),
                       what=f"split-K M={M} N={N} K={K}")
    g = oracle.bf16_to_f32(y1).astype(np.float64)
    h = oracle.bf16_to_f32(y2).astype(np.float64)
    # fp32 atomics may add partials in another order: allow one bf16 ulp
    assert np.max(np.abs(g - h) / (np.abs(g) + 1e-3)) <= 2 ** -7


def test_graph_replay_matches_eager(gpu):
    """The decode stack runs from a captured HIP graph in bench.py: replays, with
    eager work in between, must reproduce the eager result every time."""
    from fastmlx_amd import ops

    rng = np.random.default_rng(77)
    # M=1 / 4 GEMVs, qmvs (M=16, narrow), qmvw with K parts and its fixup (M=32),
    # the prefill GEMM (M=96) and the wide GEMM (M=1024, 2048).
    shapes = [(1, 4096, 4096), (4, 1024, 4096), (16, 2048, 2048), (32, 4096, 4096),
              (96, 512, 1024), (1024, 1024, 1024), (2048, 4096, 1024)]
    tensors = []
    for M, N, K in shapes:
        w, s, b = make_quant(rng, (N,), K, 4, 64)
        x = make_x(rng, M, K)
        tensors.append(tuple(to_dev(t, gpu) for t in (x, w, s, b)) +
                       (torch.empty(M, N, dtype=torch.bfloat16, device=gpu),))

    def step():
        for x, w, s, b, y in tensors:
            ops.quantized_matmul(x, w, s, b, True, 64, 4, out=y)

    announce("graph capture of quantized_matmul calls")
    step()
    torch.cuda.synchronize()
    eager = [to_np(t[-1]).copy() for t in tensors]
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()  # warm the split-K workspace of the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=side):
        step()
    for rep in range(4):
        for t in tensors:
            t[-1].zero_()
        g.replay()
        torch.cuda.synchronize()
        for t, e in zip(tensors, eager):
            got = oracle_free_close(to_np(t[-1]), e)
            assert got, f"replay {rep} differs from eager"
        step()  # eager work between replays
        torch.cuda.synchronize()


def oracle_free_close(a, b):
    fa = (a.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    fb = (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return bool(np.all(np.abs(fa - fb) <= 2 ** -7 * (np.abs(fb) + 1e-3)))


def test_zero_sizes_enqueue_nothing(gpu):
    from fastmlx_amd import _lib

    lib = _lib.load()
    assert lib.fmxq_quantized_matmul(None, None, None, None, None, 0, 16, 64, True, 64, 4,
                                     None) == 0


@pytest.mark.parametrize("M,Ns,K,bits,group", [
    (1, (4096, 1024, 1024), 4096, 4, 64),   # q | k | v of the C1 stack: one grouped launch
    (1, (14336, 14336), 4096, 4, 64),       # gate | up: one launch, 4-row waves by the total
    (1, (4096,), 14336, 4, 64),             # one product, 14336-deep rows
    (1, (1030, 0, 77, 2050), 2048, 4, 64),  # four products, an empty one, ragged rows, 1 slice
    (2, (1024, 512), 4096, 4, 64),          # M = 2: one launch per product
    (1, (1024, 2048), 4096, 8, 64),         # int8: one launch per product
    (1, (1024, 520), 6144, 4, 64),          # three slices: one launch per product
])
def test_quantized_matmul_group(gpu, oracle, M, Ns, K, bits, group):
    """fmxq_quantized_matmul_group: every product checked element by element against
    the fp64 oracle and by the 2e-2 metric, and against fmxq_quantized_matmul of the
    same product (equal where both run the same wave shape, within the tolerance
    otherwise)."""
    import parity
    from fastmlx_amd import ops

    rng = np.random.default_rng(7000 + M + K + sum(Ns))
    x = make_x(rng, M, K)
    mats = [make_quant(rng, (N,), K, bits, group) for N in Ns]
    announce(f"quantized_matmul_group M={M} Ns={Ns} K={K} bits={bits}")
    dx = to_dev(x, gpu)
    dm = [tuple(to_dev(t, gpu) for t in m) for m in mats]
    ys = ops.quantized_matmul_group(dx, dm, group, bits)
    singles = [ops.quantized_matmul(dx, *m, True, group, bits) for m in dm]
    torch.cuda.synchronize()
    for i, (N, (w, s, b)) in enumerate(zip(Ns, mats)):
        got = to_np(ys[i])
        assert got.shape == (M, N)
        if N == 0:
            continue
        ref = parity.DenseRef(np.ascontiguousarray(x), w, s, b, group, bits)
        parity.check_dense(got, ref, what=f"group product {i}: M={M} N={N} K={K}")
        e = rel_err(oracle.bf16_to_f32(got), ref.mlx)
        assert e < 2e-2, e
        one = oracle.bf16_to_f32(to_np(singles[i]))
        assert rel_err(oracle.bf16_to_f32(got), one) < 2e-2


def test_quantized_matmul_group_validation(gpu):
    """Refusals before any launch: n outside 1..4, and K / w disagreeing."""
    from fastmlx_amd import ops

    rng = np.random.default_rng(3)
    x = to_dev(make_x(rng, 1, 2048), gpu)
    m = tuple(to_dev(t, gpu) for t in make_quant(rng, (64,), 2048, 4, 64))
    with pytest.raises(Exception):
        ops.quantized_matmul_group(x, [m] * 5)
    m4 = tuple(to_dev(t, gpu) for t in make_quant(rng, (64,), 4096, 4, 64))
    with pytest.raises(ValueError):
        ops.quantized_matmul_group(x, [m, m4])


def test_quantized_matmul_group_graph_replay(gpu):
    """The grouped launch (its matrix table travels in the kernel arguments) captured
    in a HIP graph: every replay, with eager calls between them, equals the eager
    result bit for bit."""
    from fastmlx_amd import ops

    rng = np.random.default_rng(11)
    x = to_dev(make_x(rng, 1, 4096), gpu)
    mats = [tuple(to_dev(t, gpu) for t in make_quant(rng, (N,), 4096, 4, 64))
            for N in (4096, 1024, 1024)]
    outs = [torch.empty(1, w.shape[0], dtype=torch.bfloat16, device=gpu) for w, _, _ in mats]

    def step():
        ops.quantized_matmul_group(x, mats, 64, 4, outs=outs)

    announce("graph capture of quantized_matmul_group")
    step()
    torch.cuda.synchronize()
    eager = [to_np(y).copy() for y in outs]
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=side):
        step()
    for rep in range(3):
        for y in outs:
            y.zero_()
        g.replay()
        torch.cuda.synchronize()
        for y, e in zip(outs, eager):
            assert np.array_equal(to_np(y), e), f"replay {rep} differs from eager"
        step()
        torch.cuda.synchronize()
