"""GPU parity of the array-handle layer (include/fmx.h) and the model-side mirror.

Each op goes through the mlx-c-shaped entry points with MLX shape semantics
(leading axes flattened, gather_qmm batch broadcasting, implicit aranges) and is
checked against the oracle on the same bytes: dequantize bit-exact, products to
the per-element fp64 bound and the 2e-2 metric (tests/parity.py).  Covers the reference's two gather_qmm call shapes
(switch_glu.go:124-130 unsorted x [B,L,1,1,D] with rhs [B,L,k]; :135-152 sorted
x [S,1,D] with rhs [S]) and the general broadcast forms MLX allows.
"""
import numpy as np
import pytest

import parity
from gpu_util import announce
from synth import make_quant, make_x, topk_uniform

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fx(gpu):
    from fastmlx_amd import mlxgo

    return mlxgo


def A(fx, a, dtype=None):
    return fx.Array.from_numpy(a, dtype)


def BF(fx, a):
    return fx.Array.from_numpy(a, fx.Dtype.BFLOAT16)


def quant_arrays(fx, q):
    w, s, b = q
    return A(fx, w), BF(fx, s), BF(fx, b)


def f32(oracle, h):
    return oracle.bf16_to_f32(h)


@pytest.mark.parametrize("lead,N,K,bits", [((2, 3), 256, 512, 4), ((1, 40), 128, 256, 8),
                                           ((7,), 64, 4096, 4)])
def test_quantized_matmul_leading_axes(fx, oracle, lead, N, K, bits):
    rng = np.random.default_rng(N + K + bits)
    q = make_quant(rng, (N,), K, bits)
    x = make_x(rng, *lead, K)
    announce(f"fmx quantized_matmul lead={lead} N={N} K={K} bits={bits}")
    y = fx.quantized_matmul(BF(fx, x), *quant_arrays(fx, q), True, 64, bits)
    assert y.shape() == [*lead, N] and y.dtype() == fx.Dtype.BFLOAT16
    ref = parity.DenseRef(x.reshape(-1, K), *q, 64, bits)
    parity.check_dense(y.to_numpy().reshape(-1, N), ref)
    # ToFloat32 widens bf16 exactly
    assert np.array_equal(y.to_float32().reshape(-1, N), f32(oracle, y.to_numpy()).reshape(-1, N))


def test_quantized_matmul_bias(fx, oracle):
    rng = np.random.default_rng(3)
    N, K = 96, 256
    q = make_quant(rng, (N,), K)
    x = make_x(rng, 3, K)
    bias = make_x(rng, N)
    announce("fmx quantized_matmul_bias")
    y = fx.quantized_matmul_bias(BF(fx, x), *quant_arrays(fx, q), BF(fx, bias), True, 64, 4)
    parity.check_dense(y.to_numpy(), parity.DenseRef(x, *q, 64, 4), bias16=bias)


def test_dequantize_batched_bit_exact(fx, oracle):
    rng = np.random.default_rng(4)
    for bits in (4, 8):
        q = make_quant(rng, (3, 32), 256, bits)
        announce(f"fmx dequantize [3,32,*] bits={bits}")
        got = fx.dequantize(*quant_arrays(fx, q), 64, bits).to_numpy()
        want = oracle.dequantize(q[0].reshape(96, -1), q[1].reshape(96, -1), q[2].reshape(96, -1),
                                 64, bits)
        assert got.shape == (3, 32, 256)
        assert np.array_equal(got.reshape(96, 256), want)


@pytest.mark.parametrize("idx_dtype", [np.int32, np.int64, np.uint16])
def test_dequantize_rows_is_qembed(fx, oracle, idx_dtype):
    rng = np.random.default_rng(5)
    V, D = 50, 256
    q = make_quant(rng, (V,), D)
    idx = rng.integers(0, V, size=(2, 5)).astype(idx_dtype)
    announce(f"fmx dequantize_rows idx {np.dtype(idx_dtype).name}")
    got = fx.dequantize_rows(*quant_arrays(fx, q), A(fx, idx), 64, 4).to_numpy()
    table = oracle.dequantize(*q, 64, 4)
    assert got.shape == (2, 5, D)
    assert np.array_equal(got, table[idx.astype(np.int64)])


def test_dequantize_rows_bad_index(fx, oracle):
    rng = np.random.default_rng(6)
    q = make_quant(rng, (8,), 128)
    idx = np.array([1, 8, -1, 3], dtype=np.int32)
    announce("fmx dequantize_rows out-of-range")
    out = fx.dequantize_rows(*quant_arrays(fx, q), A(fx, idx), 64, 4)
    with pytest.raises(fx.MLXError) as e:
        out.eval()
    assert e.value.code == 4
    got = out.to_numpy()  # the flag was cleared by the failed eval
    table = oracle.dequantize(*q, 64, 4)
    assert np.array_equal(got[[0, 3]], table[[1, 3]])
    assert not got[1].any() and not got[2].any()


def _gather_ref(oracle, x_items, q, xi, ei, bits=4):
    """fp64 references over flat items: y[i] = x_items[xi[i]] (Mx x K) . deq(W[ei[i]])^T."""
    n_items, Mx, K = x_items.shape
    xi, ei = np.asarray(xi).ravel(), np.asarray(ei).ravel()
    xrow = (xi[:, None] * Mx + np.arange(Mx)[None, :]).ravel()
    erow = np.repeat(ei, Mx)
    return parity.gather_refs(x_items.reshape(-1, K), *q, xrow, erow, 64, bits)


def test_gather_qmm_unsorted_choreography(fx, oracle):
    """switch_glu.go:124-130: x [B,L,1,1,D], rhs [B,L,k] -> [B,L,k,1,N]."""
    rng = np.random.default_rng(7)
    Bsz, L, k, E, D, N = 2, 3, 4, 6, 256, 128
    q = make_quant(rng, (E, N), D)
    x = make_x(rng, Bsz, L, 1, 1, D)
    rhs = topk_uniform(rng, Bsz * L, E, k).reshape(Bsz, L, k).astype(np.int32)
    announce("fmx gather_qmm unsorted [B,L,1,1,D]")
    y = fx.gather_qmm(BF(fx, x), *quant_arrays(fx, q), None, A(fx, rhs), True, 64, 4, False)
    assert y.shape() == [Bsz, L, k, 1, N]
    xi = np.repeat(np.arange(Bsz * L), k)
    ref = _gather_ref(oracle, x.reshape(Bsz * L, 1, D), q, xi, rhs)
    parity.check_dense(y.to_numpy().reshape(-1, N), ref, what="gather_qmm")


@pytest.mark.parametrize("S", [40, 200])
def test_gather_qmm_sorted_choreography(fx, oracle, S):
    """switch_glu.go:135-152: x [S,1,D] rows already sorted, rhs [S] ascending."""
    rng = np.random.default_rng(S)
    E, D, N = 8, 512, 256
    q = make_quant(rng, (E, N), D)
    x = make_x(rng, S, 1, D)
    rhs = np.sort(rng.integers(0, E, size=S)).astype(np.uint32)
    announce(f"fmx gather_qmm sorted S={S}")
    y = fx.gather_qmm(BF(fx, x), *quant_arrays(fx, q), None, A(fx, rhs), True, 64, 4, True)
    assert y.shape() == [S, 1, N]
    ref = _gather_ref(oracle, x, q, np.arange(S), rhs)
    parity.check_dense(y.to_numpy().reshape(-1, N), ref, what="gather_qmm")


def test_gather_qmm_broadcast_lhs_rhs(fx, oracle):
    """Explicit int64 lhs [S,1] against rhs [1,k]: batch [S,k], Mx = 2 rows each."""
    rng = np.random.default_rng(9)
    X, S, k, E, D, N, Mx = 5, 6, 3, 4, 128, 64, 2
    q = make_quant(rng, (E, N), D)
    x = make_x(rng, X, Mx, D)
    lhs = rng.integers(0, X, size=(S, 1)).astype(np.int64)
    rhs = rng.integers(0, E, size=(1, k)).astype(np.int32)
    announce("fmx gather_qmm broadcast lhs/rhs")
    y = fx.gather_qmm(BF(fx, x), *quant_arrays(fx, q), A(fx, lhs), A(fx, rhs), True, 64, 4,
                      False)
    assert y.shape() == [S, k, Mx, N]
    bl, br = np.broadcast_arrays(lhs, rhs)
    ref = _gather_ref(oracle, x, q, bl, br)
    parity.check_dense(y.to_numpy().reshape(-1, N), ref, what="gather_qmm")


def test_gather_qmm_implicit_aranges(fx, oracle):
    """No lhs with x batch [1,4] vs rhs [3,4] (materialized arange), and no rhs
    with an explicit lhs (arange over w's batch)."""
    rng = np.random.default_rng(10)
    E, D, N = 4, 128, 64
    q = make_quant(rng, (E, N), D)
    x = make_x(rng, 1, 4, 1, D)
    rhs = rng.integers(0, E, size=(3, 4)).astype(np.int32)
    announce("fmx gather_qmm implicit lhs arange")
    y = fx.gather_qmm(BF(fx, x), *quant_arrays(fx, q), None, A(fx, rhs), True, 64, 4, False)
    assert y.shape() == [3, 4, 1, N]
    xi = np.broadcast_to(np.arange(4)[None, :], (3, 4))
    ref = _gather_ref(oracle, x.reshape(4, 1, D), q, xi, rhs)
    parity.check_dense(y.to_numpy().reshape(-1, N), ref, what="gather_qmm")

    x2 = make_x(rng, 6, 1, D)
    lhs = rng.integers(0, 6, size=(E,)).astype(np.int32)
    announce("fmx gather_qmm implicit rhs arange")
    y2 = fx.gather_qmm(BF(fx, x2), *quant_arrays(fx, q), A(fx, lhs), None, True, 64, 4, False)
    assert y2.shape() == [E, 1, N]
    ref2 = _gather_ref(oracle, x2, q, lhs, np.arange(E))
    parity.check_dense(y2.to_numpy().reshape(-1, N), ref2, what="gather_qmm")


def test_gather_qmm_bad_index_reported_at_eval(fx, oracle):
    rng = np.random.default_rng(11)
    E, D, N = 3, 128, 64
    q = make_quant(rng, (E, N), D)
    x = make_x(rng, 4, 1, D)
    rhs = np.array([0, 7, 1, -2], dtype=np.int32)
    announce("fmx gather_qmm bad rhs")
    y = fx.gather_qmm(BF(fx, x), *quant_arrays(fx, q), None, A(fx, rhs), True, 64, 4, False)
    with pytest.raises(fx.MLXError) as e:
        y.eval()
    assert e.value.code == 4
    got = y.to_numpy().reshape(4, N)
    assert not got[1].any() and not got[3].any()


@pytest.mark.parametrize("L,k", [(2, 3), (32, 2)])
def test_switch_glu_via_handles_and_fb(fx, oracle, L, k):
    from fastmlx_amd.models import FB, QLinear

    rng = np.random.default_rng(L * 10 + k)
    E, D, I = 8, 128, 64
    gate, up = make_quant(rng, (E, I), D), make_quant(rng, (E, I), D)
    down = make_quant(rng, (E, D), I)
    x = make_x(rng, 1, L, D)
    inds = topk_uniform(rng, L, E, k).reshape(1, L, k).astype(np.int32)
    ql = lambda t: QLinear(*quant_arrays(fx, t), group_size=64, bits=4)
    announce(f"fmx switch_glu L={L} k={k} (slots {L * k})")
    b = FB()
    y = b.switch_glu_for(BF(fx, x), ql(gate), ql(up), ql(down), A(fx, inds))
    assert b.err is None and y.shape() == [1, L, k, D]
    sref = parity.SwitchRef(x.reshape(L, D), inds.reshape(L, k), gate, up, down)
    parity.check_switch(y.to_numpy().reshape(L, k, D), sref)


def test_fb_qlinear_qembed_combine(fx, oracle):
    from fastmlx_amd.models import FB, QLinear

    rng = np.random.default_rng(12)
    N, K, V = 128, 256, 40
    q = make_quant(rng, (N,), K)
    tq = make_quant(rng, (V,), K)
    x = make_x(rng, 1, 2, K)
    b = FB(fx.default_stream())
    y = b.qlinear(BF(fx, x), QLinear(*quant_arrays(fx, q), group_size=64, bits=4))
    idx = np.array([[3, 39, 0]], dtype=np.int32)
    e = b.qembed(QLinear(*quant_arrays(fx, tq), group_size=64, bits=4), A(fx, idx))
    yk = make_x(rng, 2, 3, 4, 64)
    wk = oracle.f32_to_bf16(rng.uniform(0, 1, (2, 3, 4)).astype(np.float32))
    c = b.moe_combine(BF(fx, yk), BF(fx, wk))
    announce("fmx FB qlinear/qembed/moe_combine")
    assert b.err is None
    parity.check_dense(y.to_numpy().reshape(2, N), parity.DenseRef(x[0], *q, 64, 4))
    assert np.array_equal(e.to_numpy()[0], oracle.dequantize(*tq, 64, 4)[idx[0]])
    r16 = lambda v: f32(oracle, oracle.f32_to_bf16(v.astype(np.float32)))
    want = r16(r16(f32(oracle, yk) * f32(oracle, wk)[..., None]).sum(2))
    assert c.shape() == [2, 3, 64]
    assert np.all(np.abs(f32(oracle, c.to_numpy()) - want) <= 2.0 ** -7 * np.abs(want) + 1e-30)


def test_buffer_cache_and_cross_stream(fx, oracle):
    """A freed result's buffer is reused by the next result of the same size on
    the same stream; a result made on one stream is read correctly on another."""
    rng = np.random.default_rng(13)
    N, K = 256, 512
    q = make_quant(rng, (N,), K)
    qa = quant_arrays(fx, q)
    x = BF(fx, make_x(rng, 4, K))
    s1, s2 = fx.new_stream(), fx.new_stream()
    announce("fmx buffer cache + cross-stream")
    y1 = fx.quantized_matmul(x, *qa, True, 64, 4, s1)
    p1 = y1.device_ptr()
    y1.free()
    y2 = fx.quantized_matmul(x, *qa, True, 64, 4, s1)
    assert y2.device_ptr() == p1
    # y2 (made on s1) feeds a product on s2: the layer fences s2 on s1
    w2 = make_quant(rng, (64,), N)
    z = fx.quantized_matmul(y2, *quant_arrays(fx, w2), True, 64, 4, s2)
    s2.synchronize()
    parity.check_dense(y2.to_numpy(), parity.DenseRef(x.to_numpy(), *q, 64, 4))
    parity.check_dense(z.to_numpy(), parity.DenseRef(y2.to_numpy(), *w2, 64, 4))
    # replacing a live result handle in place (mlx-c set semantics) keeps it valid
    y2.free()
    z.free()


def test_fb_moe_layer_router_switch_combine(fx, oracle):
    """A Qwen3-Next MoE block through the handle layer (qwen3next_forward.go:510-525,
    routed part): router logits from qlinear, softmax top-k router, switchGLU over
    the picked experts, weighted combine; against the oracle on the same bytes."""
    from fastmlx_amd.models import FB, QLinear

    rng = np.random.default_rng(77)
    E, D, I, k, L = 16, 128, 64, 4, 6
    router = make_quant(rng, (E,), D)
    gate, up = make_quant(rng, (E, I), D), make_quant(rng, (E, I), D)
    down = make_quant(rng, (E, D), I)
    x = make_x(rng, 1, L, D)
    ql = lambda t: QLinear(*quant_arrays(fx, t), group_size=64, bits=4)
    announce(f"fmx MoE block L={L} E={E} k={k}")
    b = FB()
    logits = b.qlinear(BF(fx, x), ql(router))
    inds, scores = b.route_softmax(logits, k, True)
    y = b.switch_glu_for(BF(fx, x), ql(gate), ql(up), ql(down), inds)
    out = b.moe_combine(y, scores)
    assert b.err is None
    assert inds.shape() == [1, L, k] and scores.shape() == [1, L, k] and out.shape() == [1, L, D]
    lg = f32(oracle, logits.to_numpy().reshape(L, E))
    oi, ow = oracle.route_softmax_topk(lg, k, norm=True)
    assert np.array_equal(inds.to_numpy().view(np.uint32).reshape(L, k), oi)
    got_w = f32(oracle, scores.to_numpy().reshape(L, k))
    assert np.allclose(got_w, ow, rtol=2 ** -8, atol=1e-6)
    sref = parity.SwitchRef(x.reshape(L, D), oi, gate, up, down)
    ys = y.to_numpy().reshape(L, k, D)
    parity.check_switch(ys, sref)
    near = parity.nearest(ys, sref)
    parity.combine_check(out.to_numpy().reshape(L, D), near,
                         parity.switch_bound(near, near, sref.hscale),
                         scores.to_numpy().reshape(L, k))


def test_fb_route_experts_reference_vectors(fx):
    """DeepSeek routeExperts through the handle layer on the reference's routing
    vectors (compute/models/deepseekv3_test.go:130-163)."""
    import json
    import os

    from fastmlx_amd.models import FB

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                        "deepseek_routing.json")
    with open(path) as f:
        cases = json.load(f)["routing"]
    b = FB()
    for c in cases:
        announce(f"fmx route_experts {c['label']}")
        g = A(fx, np.array([[c["gates"]]], np.float32))
        bias = A(fx, np.array(c["bias"], np.float32))
        inds, w = b.route_experts(g, bias, c["top_k"], c["n_group"], c["topk_group"],
                                  c["routed_scaling_factor"], c["norm_topk_prob"])
        assert b.err is None and inds.shape() == [1, 1, c["top_k"]]
        got = dict(zip(inds.to_numpy().view(np.uint32).ravel().tolist(),
                       w.to_numpy().view(np.float32).ravel().tolist()))
        want = dict(zip(c["inds"], c["scores"]))
        assert set(got) == set(want)
        for e, v in want.items():
            assert abs(got[e] - v) <= 1e-5 * abs(v)
