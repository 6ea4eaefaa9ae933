"""Pin the CPU oracle (oracle/ponni_oracle.cpp) before trusting it.

Every check is one the reference itself makes or one the mathematics fixes:
  - the reference's known-answer tests (unit/core/test_core_unit.cpp,
    unit/core/test_template_coverage.cpp, unit/performance_benchmark);
  - the reference's scratch-planning answers (tmp1 / tmp2 widths);
  - binary16 / bfloat16 rounding against numpy / torch conversions;
  - random chains of every layer kind against a vectorized float64 numpy
    evaluation (tests/numpy_ref.py) at several widths and batch sizes.
"""
import math

import numpy as np
import pytest

import oracle
import ponni_amd as P
from tests import numpy_ref


@pytest.fixture(scope="module", autouse=True)
def _built():
    oracle.build()


def run(layers, x, mode=oracle.MODE_F32):
    return oracle.forward(layers, np.asarray(x, dtype=np.float64 if mode == oracle.MODE_F64 else np.float32), mode)


def test_first_model_known_answer():
    # test_core_unit.cpp:200-221: 2x2 ones, bias 1, LeakyRelu(0.1), x = (1, 2) -> (4, 4)
    layers = [P.Matvec(np.ones((2, 2))), P.Bias(np.ones(2)), P.LeakyRelu(2, 0.1)]
    y = run(layers, [[1.0], [2.0]])
    assert np.allclose(y[:, 0], [4.0, 4.0], atol=1e-6)
    tmp, _ = oracle.plan_widths(layers)
    assert tmp == [0, 0]  # a single fused block needs no scratch (test_core_unit.cpp:220-221)


def test_four_block_fused_network():
    # test_core_unit.cpp:262-326: widths 5/3/7, closed form at :310-318, tol 1e-4
    layers = [P.Matvec(np.ones((2, 5))), P.Bias(np.full(5, 0.5)), P.Relu(5), P.Tanh(5),
              P.Matvec(np.ones((5, 3))), P.Bias(np.full(3, -0.25)), P.Sigmoid(3),
              P.Matvec(np.ones((3, 7))), P.Bias(np.full(7, 0.1)), P.LeakyRelu(7, 0.2),
              P.Matvec(np.ones((7, 2))), P.Bias(np.full(2, -0.2)), P.HardSwish(2)]
    x = np.array([[1.0, -2.0, 0.0], [2.0, 0.5, 0.0]])
    y = run(layers, x)
    for b in range(3):
        s = x[0, b] + x[1, b]
        h1 = math.tanh(max(0.0, s + 0.5))
        d2 = 5 * h1 - 0.25
        h2 = 1 / (1 + math.exp(-d2))
        d3 = 3 * h2 + 0.1
        h3 = d3 if d3 > 0 else 0.2 * d3
        d4 = 7 * h3 - 0.2
        e = 0.0 if d4 <= -3 else d4 if d4 >= 3 else d4 * (d4 + 3) / 6
        assert abs(y[0, b] - e) <= 1e-4 and abs(y[1, b] - e) <= 1e-4
    tmp, _ = oracle.plan_widths(layers)
    assert tmp == [7, 3]  # test_core_unit.cpp:304-307


def test_softmax_barrier_between_blocks():
    # test_core_unit.cpp:331-378 -> (tanh 1, 0); tmp1 = 3, no tmp2
    layers = [P.Matvec(np.ones((2, 3))), P.Bias([0.0, 1.0, 2.0]), P.Relu(3), P.Softmax(3),
              P.Matvec(np.ones((3, 2))), P.Bias([0.0, -1.0]), P.Tanh(2)]
    y = run(layers, np.full((2, 2), 0.5))
    assert np.allclose(y[0], math.tanh(1.0), atol=1e-5) and np.allclose(y[1], 0.0, atol=1e-5)
    tmp, _ = oracle.plan_widths(layers)
    assert tmp == [3, 0]


def test_matvec_in_out_layout():
    # test_core_unit.cpp:516-546: W = 10..15 as [2, 3], x = (1, 2) -> out0 = 36, out2 = 42
    layers = [P.Matvec(np.arange(10.0, 16.0).reshape(2, 3))]
    y = run(layers, [[1.0], [2.0]])
    assert y[0, 0] == 36.0 and y[2, 0] == 42.0 and y[1, 0] == 39.0


ACTS = [
    (P.Relu(3), [0.0, 0.0, 2.0], 1e-5),
    (P.LeakyRelu(3, 0.1), [-0.1, 0.0, 2.0], 1e-5),
    (P.Elu(3), [math.exp(-1) - 1, 0.0, 2.0], 1e-5),
    (P.Selu(3), [1.0507009873554804934 * 1.6732632423543772848 * (math.exp(-1) - 1), 0.0,
                 1.0507009873554804934 * 2], 2e-5),
    (P.Gelu(3), [-0.5 * (1 - math.erf(1 / math.sqrt(2))), 0.0, 1 + math.erf(math.sqrt(2))], 2e-5),
    (P.Gelu(3, True), [-0.158808, 0.0, 1.954598], 2e-5),
    (P.Silu(3), [-1 / (1 + math.e), 0.0, 2 / (1 + math.exp(-2))], 2e-5),
    (P.Sigmoid(3), [1 / (1 + math.e), 0.5, 1 / (1 + math.exp(-2))], 2e-5),
    (P.Tanh(3), [math.tanh(-1), 0.0, math.tanh(2)], 1e-5),
    (P.Softplus(3, 2.0), [0.5 * math.log(1 + math.exp(-2)), 0.5 * math.log(2), 0.5 * math.log(1 + math.exp(4))], 2e-5),
    (P.HardSigmoid(3, 0.2, 0.5), [0.3, 0.5, 0.9], 1e-5),
    (P.HardSwish(3), [-2 / 6, 0.0, 10 / 6], 1e-5),
    (P.Mish(3), [-math.tanh(math.log(1 + math.exp(-1))), 0.0, 2 * math.tanh(math.log(1 + math.exp(2)))], 2e-5),
]


@pytest.mark.parametrize("layer,expected,tol", ACTS, ids=[a[0].label + str(i) for i, a in enumerate(ACTS)])
def test_activation_known_answers(layer, expected, tol):
    # test_core_unit.cpp:627-703: every activation at x in {-1, 0, 2}
    y = run([layer], [[-1.0], [0.0], [2.0]])
    assert np.allclose(y[:, 0], expected, atol=tol)


def test_softmax_and_log_softmax_known_answers():
    s = math.exp(-3) + math.exp(-2) + 1
    y = run([P.Softmax(3)], [[-1.0], [0.0], [2.0]])
    assert np.allclose(y[:, 0], [math.exp(-3) / s, math.exp(-2) / s, 1 / s], atol=1e-5)
    lse = math.log(s) + 2
    y = run([P.LogSoftmax(3)], [[-1.0], [0.0], [2.0]])
    assert np.allclose(y[:, 0], [-1 - lse, -lse, 2 - lse], atol=1e-5)


def test_layer_norm_exact():
    # test_core_unit.cpp:705-771 checks mean ~ 0; pin the values exactly in fp64
    x = np.array([[1.0], [2.0], [3.0], [4.0]])
    y = run([P.LayerNorm(4)], x, oracle.MODE_F64)
    mu, var = 2.5, 1.25
    assert np.allclose(y[:, 0], (x[:, 0] - mu) / math.sqrt(var + 1e-5), rtol=0, atol=1e-14)
    g, b = np.array([2.0, 1.0, 0.5, -1.0]), np.array([0.5, 0.0, -0.5, 1.0])
    y = run([P.LayerNorm(g, b, 1e-3)], x, oracle.MODE_F64)
    assert np.allclose(y[:, 0], g * (x[:, 0] - mu) / math.sqrt(var + 1e-3) + b, atol=1e-14)


def test_min_max_norm():
    # test_core_unit.cpp:774-812: (2, 5, 8) over [-1, 1] -> (-1, 0, 1)
    y = run([P.MinMaxNorm(3, -1.0, 1.0)], [[2.0], [5.0], [8.0]])
    assert np.allclose(y[:, 0], [-1.0, 0.0, 1.0], atol=1e-5)


def test_projection_skip():
    # test_core_unit.cpp:814-872: current (1,2,3), saved (4,5) -> (5.1, 7.2, 7.8)
    w = np.array([[1.0, 0.0, 0.5], [0.0, 1.0, 0.5]])
    b = np.array([0.1, 0.2, 0.3])
    layers = [P.Save_State(0, 2), P.Matvec(np.array([[0.25, 0.0, 0.0], [0.0, 0.4, 0.6]])),
              P.Binop_Projection_Add(0, w, b)]
    y = run(layers, [[4.0], [5.0]])
    assert np.allclose(y[:, 0], [5.1, 7.2, 7.8], atol=1e-5)


def test_leading_save_and_projection_residual():
    # test_template_coverage.cpp:414-470: (-2, 3) -> (-2, 6) through Add and through identity projection
    x = [[-2.0], [3.0]]
    y = run([P.Save_State(0, 2), P.Relu(2), P.Binop_Add(0, 2)], x)
    assert np.allclose(y[:, 0], [-2.0, 6.0])
    y = run([P.Save_State(0, 2), P.Relu(2), P.Binop_Projection_Add(0, np.eye(2), np.zeros(2), False)], x)
    assert np.allclose(y[:, 0], [-2.0, 6.0])


def test_multiple_saved_slots():
    # test_template_coverage.cpp:471-500: -> {0, 6, -2, 6, -2, 3}
    layers = [P.Save_State(0, 2), P.Relu(2), P.Binop_Concatenate(0, 2, 4, True), P.Save_State(1, 4), P.Relu(4),
              P.Binop_Add(1, 4), P.Binop_Concatenate(0, 4, 6, True)]
    y = run(layers, [[-2.0], [3.0]])
    assert np.allclose(y[:, 0], [0.0, 6.0, -2.0, 6.0, -2.0, 3.0])
    _, saved = oracle.plan_widths(layers)
    assert saved[:2] == [2, 4]


def test_concatenate_before():
    # test_core_unit.cpp:432-447: after=false puts the saved rows first
    layers = [P.Save_State(0, 2), P.Matvec(np.array([[1.0, 0.0], [0.0, 1.0]]) * 1.0),
              P.Binop_Concatenate(0, 2, 4, False)]
    y = run(layers, [[10.0], [20.0]])
    assert np.allclose(y[:, 0], [10.0, 20.0, 10.0, 20.0])
    layers = [P.Save_State(0, 2), P.Matvec(np.array([[2.0, 0.0], [0.0, 2.0]])), P.Binop_Concatenate(0, 2, 4, False)]
    y = run(layers, [[10.0], [20.0]])
    assert np.allclose(y[:, 0], [10.0, 20.0, 20.0, 40.0])


def test_performance_benchmark_closed_form():
    # unit/performance_benchmark/performance_benchmark.cpp:17-53: mean output 15.4
    layers = [P.Matvec(np.ones((8, 8))), P.Bias(np.ones(8)), P.LeakyRelu(8, 0.1),
              P.Matvec(np.ones((8, 8))), P.Bias(np.ones(8)), P.LeakyRelu(8, 0.1)]
    y = run(layers, np.full((8, 4096), 0.1))
    assert abs(y.mean() - 15.4) <= 1e-3


def test_half_rounding_matches_numpy():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(2000) * 10.0 ** rng.integers(-9, 5, 2000),
        [0.0, -0.0, 65504.0, 65519.9, 65520.0, 1e-8, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -14,
         1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, -(1.0 + 2.0 ** -11)],
    ]).astype(np.float32)
    got = np.array([oracle.round_half(float(v)) for v in vals], dtype=np.float32)
    want = vals.astype(np.float16).astype(np.float32)
    assert np.array_equal(got, want)


def test_two_half_known_answers():
    # unit/core/test_core_unit.cpp:1023-1058: (2, -3) + (4, 5) = (6, 2);
    # fma((2, -3), (4, 5), (1, 2)) = (9, -13)
    assert oracle.add_half(2.0, 4.0) == 6.0 and oracle.add_half(-3.0, 5.0) == 2.0
    assert oracle.fma_half(2.0, 4.0, 1.0) == 9.0 and oracle.fma_half(-3.0, 5.0, 2.0) == -13.0


def _f16(v):
    return np.asarray(v, dtype=np.float64).astype(np.float16).astype(np.float64)


def test_fma_half_rounds_once():
    """TwoHalf::fma is __hfma2 on the device (ponni_TwoHalf.h:97-105): a * b + c
    rounded once to binary16.  numpy's float64 -> float16 conversion of the
    exact result is the reference rounding; the set includes cases where
    rounding to fp32 first and then to fp16 gives a different answer, so a
    double rounding fails here."""
    rng = np.random.default_rng(5)
    a, b, c = (_f16(rng.standard_normal(4000) * 4) for _ in range(3))
    # 2^-11 (1 + 2^-10) * (1 - 2^-10) + (1 + 2^-10) = 1 + 2^-10 + 2^-11 - 2^-31:
    # just below the tie between 1 + 2^-10 and 1 + 2^-9, so it rounds down
    # once; fp32 lands on the tie and then rounds to the even 1 + 2^-9.
    a = np.concatenate([a, [2.0 ** -11 * (1 + 2.0 ** -10)]])
    b = np.concatenate([b, [1 - 2.0 ** -10]])
    c = np.concatenate([c, [1 + 2.0 ** -10]])
    exact = a * b + c  # exact: a * b has at most 22 significant bits
    double = exact.astype(np.float32).astype(np.float16).astype(np.float64)
    want = _f16(exact)
    assert (double != want).any()
    got = np.array([oracle.fma_half(float(x), float(y), float(z)) for x, y, z in zip(a, b, c)])
    assert np.array_equal(got, want)


def _half2_chain(layers, x, fused):
    """Whole-batch numpy evaluation of a Matvec / Bias / Relu chain in binary16
    arithmetic: fused -> each step of the dot product one rounded fma (the
    generated half2 chain); else the product and the sum rounded separately
    (template half_t)."""
    v = _f16(x)
    for l in layers:
        if l.kind == P._abi.LAYER_MATVEC:
            w = _f16(l.params.reshape(l.n_in, l.n_out))
            s = np.zeros((l.n_out, v.shape[1]))
            for k in range(l.n_in):  # ascending k, ponni_Matvec.h:74-78
                p = w[k][:, None] * v[k][None, :]
                s = _f16(p + s) if fused else _f16(_f16(p) + s)
            v = s
        elif l.kind == P._abi.LAYER_BIAS:
            v = _f16(v + _f16(l.params)[:, None])
        else:
            v = np.maximum(v, 0.0)
    return v


@pytest.mark.parametrize("mode", ["half2", "half_t"])
def test_fp16_chain_modes_match_numpy_exactly(mode):
    rng = np.random.default_rng(17)
    layers = [P.Matvec(rng.standard_normal((12, 24)) * 0.4), P.Bias(rng.uniform(-0.5, 0.5, 24)), P.Relu(24),
              P.Matvec(rng.standard_normal((24, 7)) * 0.3), P.Bias(rng.uniform(-0.5, 0.5, 7))]
    x = _f16(rng.standard_normal((12, 300)) * 3)  # fp16 inputs, as the half models take them
    fused = mode == "half2"
    got = run(layers, x, oracle.MODE_F16_HALF2 if fused else oracle.MODE_F16_CHAIN)
    want = _half2_chain(layers, x, fused)
    assert np.array_equal(got, want)
    other = _half2_chain(layers, x, not fused)
    assert not np.array_equal(other, want)  # the two roundings are told apart


def test_fp16_chain_tanh_is_fp32_of_the_half_value():
    # ponni_TwoHalf.h:148-150: tanh of each lane in fp32, rounded to half.
    x = np.linspace(-6, 6, 4001)
    got = run([P.Tanh(1)], x[None, :], oracle.MODE_F16_HALF2)[0]
    want = _f16(np.tanh(_f16(x).astype(np.float32)))
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -14))) - 10)
    assert (np.abs(got - want) <= ulp).all()
    assert (got == want).mean() > 0.999


def test_bf16_rounding_matches_torch():
    import torch

    rng = np.random.default_rng(1)
    vals = (rng.standard_normal(3000) * 10.0 ** rng.integers(-20, 20, 3000)).astype(np.float32)
    got = np.array([oracle.round_bf16(float(v)) for v in vals], dtype=np.float32)
    want = torch.from_numpy(vals).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(got, want)


def random_chain(rng, width, depth, kinds="all"):
    """A random valid chain mixing dense blocks, every pointwise layer and barriers."""
    pointwise = [lambda n: P.Relu(n), lambda n: P.LeakyRelu(n, 0.05), lambda n: P.Elu(n, 0.7), lambda n: P.Selu(n),
                 lambda n: P.Gelu(n), lambda n: P.Gelu(n, True), lambda n: P.Silu(n), lambda n: P.Sigmoid(n),
                 lambda n: P.Tanh(n), lambda n: P.Softplus(n, 1.5), lambda n: P.HardSigmoid(n, 0.3, 0.4),
                 lambda n: P.HardSwish(n), lambda n: P.Mish(n)]
    n = width
    layers = [P.Save_State(0, n)]
    for d in range(depth):
        m = int(rng.integers(max(2, width // 2), width + 1))
        layers += [P.Matvec(rng.standard_normal((n, m)) / math.sqrt(n)), P.Bias(rng.uniform(-0.2, 0.2, m))]
        layers.append(pointwise[int(rng.integers(len(pointwise)))](m))
        n = m
        choice = int(rng.integers(6))
        if choice == 0:
            layers.append(P.LayerNorm(rng.uniform(0.5, 1.5, n), rng.uniform(-0.2, 0.2, n), 1e-5))
        elif choice == 1:
            layers.append(P.Binop_Projection_Add(0, rng.standard_normal((width, n)) * 0.2, rng.uniform(-0.1, 0.1, n)))
        elif choice == 2:
            layers += [P.Save_State(1, n), P.Tanh(n), P.Binop_Add(1, n)]
        elif choice == 3 and n + width <= 2 * width:
            after = bool(rng.integers(2))
            layers.append(P.Binop_Concatenate(0, n, n + width, after))
            n = n + width
        elif choice == 4:
            layers.append(P.MinMaxNorm(n, -1.0, 2.0))
    layers += [P.Matvec(rng.standard_normal((n, 5)) / math.sqrt(n)), P.Softmax(5)]
    return layers


@pytest.mark.parametrize("seed", range(12))
def test_random_chains_match_numpy_fp64(seed):
    rng = np.random.default_rng(100 + seed)
    width = [3, 8, 17, 40][seed % 4]
    layers = random_chain(rng, width, 3 + seed % 3)
    x = rng.standard_normal((width, 37))
    want = numpy_ref.evaluate(layers, x)
    got64 = run(layers, x, oracle.MODE_F64)
    assert np.allclose(got64, want, rtol=1e-11, atol=1e-12)
    got32 = run(layers, x, oracle.MODE_F32)
    assert np.abs(got32 - want).max() < 1e-4


def test_fp16_modes_are_close_to_fp64():
    rng = np.random.default_rng(7)
    layers = [P.Matvec(rng.standard_normal((16, 32)) * 0.25), P.Bias(rng.uniform(-0.1, 0.1, 32)), P.Tanh(32),
              P.Matvec(rng.standard_normal((32, 8)) * 0.2)]
    x = (rng.standard_normal((16, 64))).astype(np.float16).astype(np.float32)
    want = numpy_ref.evaluate(layers, x.astype(np.float64))
    for mode, tol in [(oracle.MODE_F16_OPERANDS, 5e-3), (oracle.MODE_BF16_OPERANDS, 4e-2), (oracle.MODE_F16_CHAIN, 1e-2)]:
        got = run(layers, x, mode)
        rel = np.linalg.norm(got - want) / np.linalg.norm(want)
        assert rel < tol, (mode, rel)
    # fp16-operand results are exactly representable in binary16
    got = run(layers, x, oracle.MODE_F16_OPERANDS)
    assert np.array_equal(got, got.astype(np.float16).astype(np.float32))


def reference_mid_chain_concat_before(state, saved):
    """What the reference executor returns for a mid-chain
    Binop_Concatenate(after=false): the barrier is in place
    (overwrite_input = true, src/layers/ponni_Binop_Concatenate.h:17), so
    compute_all_outputs gets the same tmp buffer as input and output
    (src/ponni_Inference.h:515-541) and writes it row by row
    (ponni_Binop_Concatenate.h:76-81): out[i] = i < n2 ? saved[i] : in[i - n2],
    where in[i - n2] has already been overwritten."""
    n1, n2 = len(state), len(saved)
    buf = list(state) + [0.0] * n2  # the tmp buffer (capacity-wide)
    for irow in range(n1 + n2):
        buf[irow] = saved[irow] if irow < n2 else buf[irow - n2]
    return buf


def test_mid_chain_concatenation_before_records_the_reference_defect():
    """The reference's in-place [saved; current] loses the current rows: every
    row repeats the saved state with period n2.  This build (every kernel
    family and the oracle) returns the layer's documented [saved; current]."""
    state, saved = [1.0, 2.0, 3.0], [10.0, 20.0]
    assert reference_mid_chain_concat_before(state, saved) == [10.0, 20.0, 10.0, 20.0, 10.0]
    assert reference_mid_chain_concat_before([1.0], [10.0, 20.0, 30.0]) == [10.0, 20.0, 30.0, 10.0]
    # The oracle on a chain where the concatenation is mid-chain (the state
    # lives in tmp1 and is not the last layer): Save(x) ; Relu ; Concat(before) ; Matvec(I).
    x = np.array([[-1.0, 4.0], [2.0, -3.0]])
    layers = [P.Save_State(0, 2), P.Relu(2), P.Binop_Concatenate(0, 2, 4, False), P.Matvec(np.eye(4))]
    got = oracle.forward(layers, x, oracle.MODE_F64)
    assert got.tolist() == [[-1.0, 4.0], [2.0, -3.0], [0.0, 4.0], [2.0, 0.0]]
    ref = [reference_mid_chain_concat_before([max(v, 0.0) for v in x[:, b]], list(x[:, b])) for b in range(2)]
    assert np.array(ref).T.tolist() == [[-1.0, 4.0], [2.0, -3.0], [-1.0, 4.0], [2.0, -3.0]]


def test_non_finite_inputs_follow_the_reference_loops():
    """NaN and infinity through the oracle, against answers read off the
    reference's loops.  The running minimum / maximum of MinMaxNorm
    (ponni_MinMaxNorm.h:74-78), Softmax / LogSoftmax (ponni_Softmax.h:49-52,
    ponni_LogSoftmax.h:49-52) and the generated ReduceMax / ReduceMin /
    ReduceLogSumExp (kokkos_nn/emitter.py:502-526) starts from feature 0 and
    is replaced only on a strict comparison: a NaN in feature 0 makes it NaN,
    a NaN elsewhere is passed over.  Relu is `x > 0 ? x : 0` (NaN -> 0),
    LeakyRelu `x > 0 ? x : a x` (NaN stays NaN)."""
    from ponni_amd import graph as G
    from tests.test_graph import lowered_with_params

    nan, inf = math.nan, math.inf

    def run(layers, x, mode=oracle.MODE_F64):
        return oracle.forward(layers, np.array(x, dtype=np.float64)[:, None], mode)[:, 0]

    for mode in (oracle.MODE_F64, oracle.MODE_F32):
        mm = [P.MinMaxNorm(3, -1.0, 1.0, 0.0)]
        assert np.isnan(run(mm, [nan, 1.0, 3.0], mode)).all()
        y = run(mm, [1.0, nan, 3.0], mode)
        assert y[0] == -1.0 and np.isnan(y[1]) and y[2] == 1.0
        y = run(mm, [1.0, 3.0, nan], mode)
        assert y[0] == -1.0 and y[1] == 1.0 and np.isnan(y[2])
        y = run(mm, [1.0, inf, 3.0], mode)  # scale 2 / inf = 0: finite inputs -> out_min
        assert y[0] == -1.0 and np.isnan(y[1]) and y[2] == -1.0
        for x in ([nan, 1.0, 2.0], [1.0, nan, 2.0], [1.0, 2.0, inf], [inf, 0.0, 0.0]):
            assert np.isnan(run([P.Softmax(3)], x, mode)).all(), x
            assert np.isnan(run([P.LogSoftmax(3)], x, mode)).all(), x
        y = run([P.Softmax(3)], [0.0, -inf, 0.0], mode)
        assert y.tolist() == [0.5, 0.0, 0.5]
        assert run([P.Relu(2)], [nan, -inf], mode).tolist() == [0.0, 0.0]
        y = run([P.LeakyRelu(2, 0.5)], [nan, -inf], mode)
        assert np.isnan(y[0]) and y[1] == -inf
        assert run([P.Tanh(3)], [inf, -inf, 0.0], mode).tolist() == [1.0, -1.0, 0.0]
        assert np.isnan(run([P.Tanh(1)], [nan], mode)).all()

    g = G.GraphBuilder(3)
    x = g.input
    gr = g.finish(g.concat(g.reduce("ReduceMax", x), g.reduce("ReduceMin", x), g.reduce("ReduceLogSumExp", x)))
    layers = lowered_with_params(gr)
    assert np.isnan(run(layers, [nan, 1.0, 3.0])).all()
    y = run(layers, [1.0, nan, 3.0])  # max 3, min 1; the sum meets exp(NaN - 3)
    assert y[0] == 3.0 and y[1] == 1.0 and np.isnan(y[2])
    y = run(layers, [inf, nan, 1.0])  # max inf (log-sum-exp returns it), min 1
    assert y.tolist() == [inf, 1.0, inf]
    assert np.isnan(run(layers, [nan, inf, 1.0])).all()
    y = run(layers, [1.0, -inf, 2.0])
    assert y[0] == 2.0 and y[1] == -inf and abs(y[2] - math.log(math.e + math.e ** 2)) < 1e-14

    # The generated half2 path (16-bit modes) compares the other way round,
    # reduction = TwoHalf::maximum(reduction, value) = reduction > value ?
    # reduction : value (emitter.py:578-592, ponni_TwoHalf.h:243-251): a NaN
    # is handed on to the next feature, which then replaces it.
    for mode in (oracle.MODE_F16_OPERANDS, oracle.MODE_BF16_OPERANDS):
        assert run(layers, [nan, 1.0, 3.0], mode)[:2].tolist() == [3.0, 1.0]
        assert run(layers, [1.0, nan, 3.0], mode)[:2].tolist() == [3.0, 3.0]
        assert np.isnan(run(layers, [1.0, 3.0, nan], mode)).all()
        y = run(layers, [inf, nan, 1.0], mode)  # maximum 1: the log-sum-exp meets exp(NaN - 1)
        assert y[0] == 1.0 and y[1] == 1.0 and np.isnan(y[2])
        g4 = G.GraphBuilder(4)
        four = lowered_with_params(g4.finish(g4.reduce("ReduceMax", g4.input)))
        assert run(four, [1.0, 5.0, nan, 2.0], mode).tolist() == [2.0]
        assert run(four, [1.0, 5.0, nan, 2.0], oracle.MODE_F32).tolist() == [5.0]
