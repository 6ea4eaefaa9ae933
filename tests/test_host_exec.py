"""Host execution-space models (ponni_forward_host / ponni_plan_host_model):
the plan's GENERIC op list evaluated on the host, against the CPU oracle.

This is the reference's host instantiation of Inference
(create_inference_model(DefaultHostExecutionSpace(), HostSpace(), ...),
tests/unit/test_core_unit.cpp:380-404).  fp32 bar: relative L2 <= 1e-5 and
max-abs <= 1e-4 (scaled by max(1, max|reference|) for random chains); fp64:
1e-12.  Runs without a GPU.
"""
import ctypes

import numpy as np
import pytest

import oracle
import ponni_amd as P
from ponni_amd import _abi as A
from ponni_amd import configs as C
from ponni_amd import graph as G
from tests import test_oracle as K
from tests.test_gpu_parity import KNOWN, check_f32
from tests.test_graph import lowered_with_params, random_graph


@pytest.fixture(scope="module", autouse=True)
def _oracle_built():
    oracle.build()


@pytest.mark.parametrize("name", sorted(KNOWN))
def test_known_answers_on_host(name):
    layers, x, want = KNOWN[name]
    m = P.create_inference_model(*layers)
    got = m.forward_host(np.tile(np.asarray(x), (1, 300)))
    assert np.allclose(got, np.tile(np.asarray(want), (1, 300)), atol=1e-5), got[:, :3]


def test_reference_host_model():
    # test_core_unit.cpp:380-404: Matvec(ones 2x2) + Bias(1) + LeakyRelu(0.1) on a
    # host execution/memory space, x = (1, 2) -> (4, 4).
    m = P.create_inference_model(P.Matvec(np.ones((2, 2))), P.Bias(np.ones(2)), P.LeakyRelu(2, 0.1))
    assert np.array_equal(m.forward_host(np.array([[1.0], [2.0]])), np.array([[4.0], [4.0]], dtype=np.float32))


@pytest.mark.parametrize("dtype", ["f32", "f64"])
@pytest.mark.parametrize("seed", range(10))
def test_random_chains_on_host(seed, dtype):
    rng = np.random.default_rng(500 + seed)
    width = [3, 8, 13, 16, 24, 40, 64, 100, 128, 7][seed]
    layers = K.random_chain(rng, width, 2 + seed % 4)
    B = [1, 31, 33, 255, 257, 1000, 997, 64, 129, 513][seed]
    x = rng.standard_normal((width, B))
    m = P.create_inference_model(*layers, dtype=dtype)
    xg = x.astype(np.float32).astype(np.float64) if dtype == "f32" else x
    got = m.forward_host(xg).astype(np.float64)
    if dtype == "f32":
        check_f32(got, oracle.forward(layers, xg))
    else:
        assert np.allclose(got, oracle.forward(layers, xg, oracle.MODE_F64), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c5"])
def test_configs_on_host(name):
    cfg = C.CONFIGS[name]
    layers = cfg.layers(True)
    x = np.random.default_rng(3).standard_normal((cfg.n_in, 777)).astype(np.float32).astype(np.float64)
    got = P.create_inference_model(*layers).forward_host(x).astype(np.float64)
    check_f32(got, oracle.forward(layers, x))


@pytest.mark.parametrize("seed", [0, 1, 2, 5, 7])
def test_generated_graphs_on_host(seed):
    gr = random_graph(seed, aligned=seed % 2 == 0)
    gm = G.GeneratedModel(gr)
    x = np.random.default_rng(seed).standard_normal((gr.size(gr.inputs[0]), 300)).astype(np.float32)
    got = gm.plan("f32").forward_host(x).astype(np.float64)
    check_f32(got, oracle.forward(lowered_with_params(gr), x.astype(np.float64)))


def test_threads_and_strides_agree():
    rng = np.random.default_rng(9)
    layers = K.random_chain(rng, 24, 4)
    m = P.create_inference_model(*layers)
    B = 5000
    x = rng.standard_normal((24, B)).astype(np.float32)
    one = m.forward_host(x, threads=1)
    many = m.forward_host(x, threads=7)
    assert np.array_equal(one, many)
    # Row strides larger than the batch (a column subview).
    xp = np.zeros((24, B + 5), np.float32)
    xp[:, :B] = x
    yp = np.full((one.shape[0], B + 9), np.nan, np.float32)
    A.check(A.lib().ponni_forward_host(m._plan, xp.ctypes.data, B + 5, yp.ctypes.data, B + 9, B, 3))
    assert np.array_equal(yp[:, :B], one) and np.isnan(yp[:, B:]).all()


def test_parameter_updates_are_seen_on_host():
    layers = [P.Matvec(np.ones((3, 4))), P.Bias(np.zeros(4)), P.Relu(4)]
    m = P.create_inference_model(*layers)
    x = np.ones((3, 10), np.float32)
    assert np.allclose(m.forward_host(x), 3.0)
    m.set_layer_params(0, np.full(12, 2.0))
    assert np.allclose(m.forward_host(x), 6.0)


def test_host_model_description():
    layers = [P.Save_State(0, 4), P.Matvec(np.ones((4, 6))), P.Relu(6), P.Binop_Concatenate(0, 6, 10, True)]
    m = P.create_inference_model(*layers, dtype="f64")
    d = A.DeviceModel()
    A.check(A.lib().ponni_plan_host_model(m._plan, ctypes.byref(d)))
    assert d.num_inputs == 4 and d.num_outputs == 10 and d.dtype == A.F64 and d.num_ops > 0
    assert d.num_slots == 1 and d.saved_total == 4 and d.ops and d.params
    assert ctypes.cast(d.slot_rows, ctypes.POINTER(ctypes.c_int32))[0] == 0
    # The host parameters are readable host memory: the Matvec's 24 ones.
    vals = np.ctypeslib.as_array(ctypes.cast(d.params, ctypes.POINTER(ctypes.c_double)), shape=(24,))
    assert np.array_equal(vals, np.ones(24))


def test_host_errors():
    m16 = P.create_inference_model(P.Matvec(np.ones((2, 2))), dtype="f16")
    with pytest.raises(ValueError):
        m16.forward_host(np.ones((2, 3)))
    with pytest.raises(P.PonniError) as e:
        A.check(A.lib().ponni_forward_host(m16._plan, 1, 3, 1, 3, 3, 0))
    assert e.value.status == A.PONNI_ERR_UNSUPPORTED
    m = P.create_inference_model(P.Matvec(np.ones((2, 2))))
    x = np.ones((2, 4), np.float32)
    y = np.empty((2, 4), np.float32)
    for args, status in [((x.ctypes.data, 4, y.ctypes.data, 4, 0, 0), A.PONNI_ERR_SHAPE),
                         ((x.ctypes.data, 3, y.ctypes.data, 4, 4, 0), A.PONNI_ERR_SHAPE),
                         ((None, 4, y.ctypes.data, 4, 4, 0), A.PONNI_ERR_INVALID_ARGUMENT),
                         ((x.ctypes.data, 4, y.ctypes.data, 4, 4, -1), A.PONNI_ERR_INVALID_ARGUMENT)]:
        with pytest.raises(P.PonniError) as e:
            A.check(A.lib().ponni_forward_host(m._plan, *args))
        assert e.value.status == status
