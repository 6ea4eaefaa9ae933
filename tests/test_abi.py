"""Host-side tests of libponni_hip.so: exports, plan validation, scratch planning,
.ponni I/O.  None of these touch a GPU."""
import ctypes
import os
import re
import struct

import numpy as np
import pytest

import oracle
import ponni_amd as P
from ponni_amd import _abi as A
from tests.test_oracle import random_chain

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            text = open(os.path.join(ROOT, "include", fn)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names |= set(re.findall(r"\b(ponni_\w+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    L = A.lib()
    names = declared_functions()
    assert len(names) >= 15
    for n in names:
        assert hasattr(L, n), n
    assert L.ponni_abi_version() == 1


def create(layers, dtype="f32", path="auto"):
    return P.create_inference_model(*layers, dtype=dtype, path=path)


def expect_error(layers, status, fragment, **kw):
    with pytest.raises(P.PonniError) as e:
        create(layers, **kw)
    assert e.value.status == status and fragment in e.value.message, e.value.message


def test_validation_errors():
    expect_error([P.Matvec(np.ones((2, 3))), P.Matvec(np.ones((2, 1)))], A.PONNI_ERR_INVALID_MODEL,
                 "num outputs != next layer's num inputs")
    expect_error([P.Binop_Add(0, 2)], A.PONNI_ERR_INVALID_MODEL, "cannot be first")
    expect_error([P.Relu(2), P.Binop_Add(0, 2)], A.PONNI_ERR_INVALID_MODEL, "before any Save_State")
    expect_error([P.Save_State(0, 3), P.Matvec(np.ones((3, 2))), P.Binop_Add(0, 2)], A.PONNI_ERR_INVALID_MODEL,
                 "Saved layer num inputs")
    expect_error([P.Save_State(0, 2), P.Binop_Concatenate(0, 2, 5)], A.PONNI_ERR_INVALID_MODEL, "num outputs")
    expect_error([P.Save_State(0, 2), P.Binop_Projection_Add(0, np.ones((3, 2)), np.zeros(2))],
                 A.PONNI_ERR_INVALID_MODEL, "projection weights")
    expect_error([P.Elu(2, 0.0)], A.PONNI_ERR_INVALID_MODEL, "ELU alpha")
    expect_error([P.LayerNorm(np.ones(2), np.zeros(2), 0.0)], A.PONNI_ERR_INVALID_MODEL, "epsilon")
    expect_error([P.MinMaxNorm(2, 1.0, 1.0)], A.PONNI_ERR_INVALID_MODEL, "out_max > out_min")
    expect_error([P.Save_State(4096, 2)], A.PONNI_ERR_INVALID_MODEL, "index out of range")
    expect_error([P.Save_State(-1, 2)], A.PONNI_ERR_INVALID_MODEL, "index out of range")
    expect_error([P.Matvec(np.ones((40, 40)))], A.PONNI_ERR_UNSUPPORTED, "NARROW", path="narrow")
    expect_error([P.Matvec(np.ones((2, 2)))], A.PONNI_ERR_UNSUPPORTED, "MFMA", path="mfma", dtype="f64")


def test_plan_info_and_path_selection():
    m = create([P.Matvec(np.ones((2, 3))), P.Bias(np.ones(3)), P.Relu(3), P.Matvec(np.ones((3, 1)))])
    inf = m.info()
    assert m.path == "narrow" and inf.width_class == 4 and inf.num_fused_dense_blocks == 2
    assert (inf.num_inputs, inf.num_outputs, inf.num_parameters) == (2, 1, 12)
    assert create(P.configs.CONFIGS["c2"].layers(False)).path == "fused"
    assert create(P.configs.CONFIGS["c3"].layers(False)).path == "fused"
    # F64: generated NARROW kernels up to width 16, fp64 FUSED kernels up to
    # 256, the GENERIC interpreter beyond.
    assert create([P.Matvec(np.ones((2, 2)))], dtype="f64").path == "narrow"
    assert create([P.Matvec(np.ones((40, 40)))], dtype="f64").path == "fused"
    assert create([P.Matvec(np.ones((300, 8)))], dtype="f64").path == "generic"


@pytest.mark.parametrize("seed", range(8))
def test_scratch_planning_matches_reference_rules(seed):
    rng = np.random.default_rng(seed)
    layers = random_chain(rng, [3, 8, 20, 33][seed % 4], 2 + seed % 4)
    inf = create(layers, path="generic").info()
    m = create(layers, path="generic")
    tmp, saved = oracle.plan_widths(layers)
    assert [inf.tmp1_features, inf.tmp2_features] == tmp
    assert inf.num_saved_states == len(saved)
    assert list(inf.saved_features)[:len(saved)] == saved[:8]
    assert [A.lib().ponni_plan_saved_state_size(m._plan, s) for s in range(len(saved))] == saved


def test_reference_scratch_answers():
    # test_core_unit.cpp:304-307 and :364-368
    four = [P.Matvec(np.ones((2, 5))), P.Bias(np.ones(5)), P.Relu(5), P.Tanh(5), P.Matvec(np.ones((5, 3))),
            P.Bias(np.ones(3)), P.Sigmoid(3), P.Matvec(np.ones((3, 7))), P.Bias(np.ones(7)), P.LeakyRelu(7, 0.2),
            P.Matvec(np.ones((7, 2))), P.Bias(np.ones(2)), P.HardSwish(2)]
    inf = create(four, path="generic").info()
    assert (inf.tmp1_features, inf.tmp2_features, inf.num_fused_dense_blocks) == (7, 3, 4)
    mixed = [P.Matvec(np.ones((2, 3))), P.Bias(np.ones(3)), P.Relu(3), P.Softmax(3), P.Matvec(np.ones((3, 2))),
             P.Bias(np.ones(2)), P.Tanh(2)]
    inf = create(mixed, path="generic").info()
    assert (inf.tmp1_features, inf.tmp2_features, inf.num_fused_dense_blocks) == (3, 0, 2)


def test_parameter_round_trip_and_trainable_order():
    rng = np.random.default_rng(3)
    layers = [P.Matvec(rng.standard_normal((3, 4))), P.Bias(rng.standard_normal(4), trainable=False), P.Relu(4),
              P.LayerNorm(rng.standard_normal(4), rng.standard_normal(4)),
              P.Matvec(rng.standard_normal((4, 2)))]
    m = create(layers, dtype="f64")
    for i, l in enumerate(layers):
        assert np.array_equal(m.get_layer_params(i), l.params)
    assert m.get_num_trainable_parameters() == 12 + 8 + 8
    flat = np.arange(28.0)
    m.set_trainable_parameters(flat)
    assert np.array_equal(m.get_trainable_parameters(), flat)
    assert np.array_equal(m.get_layer_params(1), layers[1].params)  # non-trainable untouched
    with pytest.raises(P.PonniError):
        A.check(A.lib().ponni_plan_set_layer_params(m._plan, 0, flat.ctypes.data, 5))


def test_forward_rejects_zero_batch_without_touching_the_device():
    m = create([P.Matvec(np.ones((2, 2)))])
    with pytest.raises(P.PonniError) as e:
        m.forward_raw(0, 0, 0, 0, 0)
    assert e.value.status == A.PONNI_ERR_SHAPE and "nonzero batch" in e.value.message


def test_fnv1a64_vectors():
    L = A.lib()
    for text, want in [(b"", 0xcbf29ce484222325), (b"a", 0xaf63dc4c8601ec8c), (b"foobar", 0x85944171f73967e8)]:
        buf = ctypes.create_string_buffer(text)
        assert L.ponni_fnv1a64(buf, len(text)) == want


def fnv(data: bytes) -> int:
    h = 0xcbf29ce484222325
    for b in data:
        h = ((h ^ b) * 0x100000001b3) & 0xFFFFFFFFFFFFFFFF
    return h


def test_template_fingerprint_format():
    # ponni_Inference.h:270-288
    layers = [P.Matvec(np.ones((2, 2))), P.Bias(np.ones(2)), P.LeakyRelu(2, 0.1)]
    m = create(layers)
    text = "ponni-template-model-v1\n0\tMatvec\t2\t2\t4\n1\tBias\t2\t2\t2\n2\tLeakyReLU\t2\t2\t0\n"
    assert m.weight_schema_fingerprint() == "fnv1a64:%016x" % fnv(text.encode())


def test_save_load_round_trip(tmp_path):
    # test_core_unit.cpp:223-238: save, zero the parameters, load, same answers
    layers = [P.Matvec(np.ones((2, 2))), P.Bias(np.ones(2)), P.LeakyRelu(2, 0.1)]
    m = create(layers)
    path = str(tmp_path / "w.ponni")
    m.save_weights(path)
    m.set_trainable_parameters(np.zeros(6))
    m.load_weights(path)
    assert np.array_equal(m.get_trainable_parameters(), np.ones(6))
    # a foreign model is rejected by fingerprint
    other = create([P.Matvec(np.ones((2, 3))), P.Bias(np.ones(3))])
    with pytest.raises(P.PonniError) as e:
        other.load_weights(path)
    assert "fingerprint" in e.value.message


def _write(path, data):
    with open(path, "wb") as f:
        f.write(bytes(data))


def safetensors_bytes(header: str, payload: int = 0):
    h = header.encode()
    return struct.pack("<Q", len(h)) + h + bytes(payload)


def test_ponni_file_rejections(tmp_path):
    # test_template_coverage.cpp:559-686 rejection matrix, through the C ABI
    L = A.lib()
    valid = str(tmp_path / "valid.ponni")
    vals = np.array([1.0, 2.0, 3.0, 4.0], dtype=np.float64)
    A.check(L.ponni_file_write_parameters(valid.encode(), b"rejection-model", vals.ctypes.data, 4, 8, b"test"))
    out = np.zeros(4)
    A.check(L.ponni_file_read_parameters(valid.encode(), b"rejection-model", out.ctypes.data, 4, 8))
    assert np.array_equal(out, vals)
    good = open(valid, "rb").read()

    def reject(label, data, fragment):
        p = str(tmp_path / (label + ".ponni"))
        _write(p, data)
        st = L.ponni_file_read_parameters(p.encode(), b"rejection-model", out.ctypes.data, 4, 8)
        msg = L.ponni_last_error().decode()
        assert st == A.PONNI_ERR_IO and fragment in msg, (label, msg)

    meta = ('"__metadata__":{"ponni.profile_version":"1","ponni.model_fingerprint":"x",'
            '"ponni.schema_fingerprint":"x","ponni.payload_checksum_fnv1a64":"x"}')
    reject("short", [0, 1, 2], "shorter")
    reject("truncated_header", good[:10], "header size")
    bad = bytearray(good)
    bad[8] = ord("[")
    reject("invalid_json", bad, "JSON")
    reject("nonobject_root", safetensors_bytes("[]"), "root must be an object")
    reject("duplicate_key", safetensors_bytes('{"x":{},"x":{}}'), "duplicate")
    reject("missing_metadata", safetensors_bytes("{}"), "no Safetensors metadata")
    reject("incomplete_descriptor", safetensors_bytes('{"x":{}}'), "incomplete")
    reject("invalid_shape", safetensors_bytes('{' + meta + ',"x":{"dtype":"F32","shape":[-1],"data_offsets":[0,4]}}', 4),
           "invalid Safetensors shape")
    reject("byte_length", safetensors_bytes('{' + meta + ',"x":{"dtype":"F64","shape":[2],"data_offsets":[0,8]}}', 8),
           "dtype, shape, and byte length")
    reject("payload_overlap", safetensors_bytes(
        '{' + meta + ',"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4]},'
        '"b":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}', 4), "hole or overlap")
    reject("nonstring_metadata", good.replace(b'"ponni.profile_version":"1"', b'"ponni.profile_version": 1 '),
           "metadata values")
    reject("unsupported_version", good.replace(b'"ponni.profile_version":"1"', b'"ponni.profile_version":"2"'),
           "profile version")
    reject("unknown_dtype", good.replace(b'"dtype":"F64"', b'"dtype":"BAD"'), "dtype, shape, and byte length")
    reject("payload_gap", safetensors_bytes(
        '{' + meta + ',"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4]},'
        '"b":{"dtype":"F32","shape":[1],"data_offsets":[5,9]}}', 9), "hole or overlap")
    reject("truncated_payload", good[:-1], "dtype, shape, and byte length")
    reject("trailing_payload", good + b"\0", "trailing bytes")
    corrupt = bytearray(good)
    corrupt[-1] ^= 1
    reject("checksum", corrupt, "checksum")
    # validation against the expected schema
    st = L.ponni_file_read_parameters(valid.encode(), b"foreign-model", out.ctypes.data, 4, 8)
    assert st == A.PONNI_ERR_IO and "fingerprint" in L.ponni_last_error().decode()
    st = L.ponni_file_read_parameters(valid.encode(), b"rejection-model", out.ctypes.data, 4, 4)
    assert st == A.PONNI_ERR_IO and "dtype mismatch" in L.ponni_last_error().decode()
    st = L.ponni_file_read_parameters(valid.encode(), b"rejection-model", out.ctypes.data, 3, 8)
    assert st == A.PONNI_ERR_IO and "shape mismatch" in L.ponni_last_error().decode()


def test_ponni_file_layout(tmp_path):
    # Header: u64 length, JSON padded with spaces to 8 bytes, payload in name order.
    L = A.lib()
    p = str(tmp_path / "layout.ponni")
    vals = np.array([1.5, -2.25, 3.0], dtype=np.float32)
    A.check(L.ponni_file_write_parameters(p.encode(), b"fp", vals.ctypes.data, 3, 4, b"template"))
    data = open(p, "rb").read()
    n = struct.unpack("<Q", data[:8])[0]
    assert n % 8 == 0 and len(data) == 8 + n + 12
    import json

    hdr = json.loads(data[8:8 + n].decode().rstrip(" "))
    md = hdr["__metadata__"]
    assert md["ponni.profile_version"] == "1" and md["ponni.model_fingerprint"] == "fp"
    assert md["ponni.target"] == "template" and md["ponni.source_framework"] == "ponni-cpp"
    assert hdr["parameters"] == {"dtype": "F32", "shape": [3], "data_offsets": [0, 12]}
    assert md["ponni.payload_checksum_fnv1a64"] == "fnv1a64:%016x" % fnv(data[8 + n:])
    schema = "ponni-tensor-schema-v1\nparameters\tF32\t3\n"
    assert md["ponni.schema_fingerprint"] == "fnv1a64:%016x" % fnv(schema.encode())
    assert np.array_equal(np.frombuffer(data[8 + n:], dtype="<f4"), vals)


@pytest.mark.parametrize("seed", range(4))
def test_fused_kernels_compile_on_the_host(seed, tmp_path, monkeypatch):
    """The generated FUSED kernel of a plan compiles with hipRTC without a GPU."""
    monkeypatch.setenv("PONNI_JIT_CACHE", str(tmp_path))
    rng = np.random.default_rng(40 + seed)
    layers = random_chain(rng, [5, 16, 33, 64][seed], 2)
    try:
        m = create(layers, path="fused")
    except P.PonniError as e:
        pytest.skip(e.message)
    src = m.kernel_source()
    assert "ponni_fused_" in src and "dense" in src
    m.compile()
    assert any(f.suffix == ".co" for f in tmp_path.iterdir())


_COMPILE_C2 = """
import sys
if sys.argv[1] == "torch":
    import torch  # brings its own hipRTC and comgr, which this process's compiles then use
import ponni_amd as P
m = P.create_inference_model(*P.configs.CONFIGS["c2"].layers(False), dtype="f32", path="fused")
m.compile()
print(min([l.split()[-1] for l in open("/proc/self/maps") if "libamd_comgr" in l] or ["none (cache hit)"]))
"""


def test_jit_cache_keyed_by_code_generator(tmp_path):
    """The on-disk kernel cache is keyed by the code generator behind hipRTC,
    not only by hipRTC's version: a process that imported torch compiles with
    torch's comgr, one that did not with the system's (both report hipRTC
    9.0), and their kernels differ in rounding, so each keeps its own object.
    A second process of either kind hits the cache."""
    import subprocess
    import sys

    env = dict(os.environ, PONNI_JIT_CACHE=str(tmp_path))

    def run(kind):
        r = subprocess.run([sys.executable, "-c", _COMPILE_C2, kind], env=env, cwd=ROOT, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        return r.stdout.strip()

    comgr_plain = run("plain")
    objects = sorted(f.name for f in tmp_path.iterdir() if f.suffix == ".co")
    assert len(objects) == 1
    comgr_torch = run("torch")
    after = sorted(f.name for f in tmp_path.iterdir() if f.suffix == ".co")
    if os.path.realpath(comgr_torch) == os.path.realpath(comgr_plain):
        assert after == objects  # one code generator: one object, found again
    else:
        assert len(after) == 2 and set(objects) < set(after)
    assert run("plain") == "none (cache hit)"  # found on disk: the compiler was never loaded
    assert sorted(f.name for f in tmp_path.iterdir() if f.suffix == ".co") == after


def _chunk_start_vmem_waits(code_object):
    """For each s_barrier of a compiled kernel followed by MFMAs before the
    next barrier: whether a vmcnt(0) wait sits between the two.  Returns
    (regions checked, regions with such a wait)."""
    import shutil
    import subprocess

    objdump = shutil.which("llvm-objdump") or "/opt/rocm/llvm/bin/llvm-objdump"
    if not os.path.exists(objdump):
        pytest.skip("llvm-objdump not found")
    out = subprocess.run([objdump, "-d", "--mcpu=gfx950", str(code_object)], capture_output=True, text=True,
                         check=True).stdout
    ins = [l.split("//")[0].strip() for l in out.splitlines()]
    ins = [l for l in ins if l and not l.endswith(":") and not l.startswith("Disassembly")]
    checked = waiting = 0
    for b in (i for i, l in enumerate(ins) if l.startswith("s_barrier")):
        j = b + 1
        while j < len(ins) and not ins[j].startswith(("v_mfma", "s_barrier", "s_endpgm")):
            j += 1
        if j < len(ins) and ins[j].startswith("v_mfma"):
            checked += 1
            waiting += any(re.match(r"s_waitcnt.*vmcnt\(0\)", l) for l in ins[b + 1:j])
    return checked, waiting


def test_half_fused_chunks_do_not_wait_for_their_own_requests(tmp_path, monkeypatch):
    """The 16-bit FUSED kernel requests weight chunk k + 2 at the start of
    chunk k, out of the compiler's wait tracking: in c4's compiled kernel no
    chunk starts (barrier, then its MFMAs) with a wait for every outstanding
    request -- only the kernel's first tile, which waits for its input rows,
    does.  (Issued through the compiler's builtin, every chunk did.)"""
    monkeypatch.setenv("PONNI_JIT_CACHE", str(tmp_path))
    m = create(P.configs.CONFIGS["c4"].layers(False), dtype="f16", path="fused")
    m.compile()
    (co,) = [f for f in tmp_path.iterdir() if f.suffix == ".co"]
    checked, waiting = _chunk_start_vmem_waits(co)
    assert checked >= 10 and waiting <= 1, (checked, waiting)


def deep_half_chain(norms=8, seed=61):
    """16-bit chain whose per-feature vectors (17 KB) outgrow the LDS left
    next to the A-fragment staging and the input rows (96 + 48 KB): 96 -> 256
    dense layer, 8 x [LayerNorm (gamma / beta: 2 KB), Tanh], 256 -> 32 dense
    layer."""
    rng = np.random.default_rng(seed)
    layers = [P.Matvec(rng.uniform(-0.15, 0.15, (96, 256))), P.Bias(rng.uniform(-0.1, 0.1, 256)), P.Tanh(256)]
    for _ in range(norms):
        layers += [P.LayerNorm(rng.uniform(0.5, 1.5, 256), rng.uniform(-0.2, 0.2, 256)), P.Tanh(256)]
    return layers + [P.Matvec(rng.uniform(-0.1, 0.1, (256, 32))), P.Bias(rng.uniform(-0.1, 0.1, 32))]


def test_half_fused_staging_and_lds_budget(tmp_path, monkeypatch):
    """16-bit FUSED kernels stage each dense layer's A fragments in 32-fragment
    chunks (a cyclic table, partial last chunks) through three LDS slots; a
    plan whose per-feature vectors would not fit next to them reads the
    vectors from global memory instead, and still compiles."""
    monkeypatch.setenv("PONNI_JIT_CACHE", str(tmp_path))
    m = create(P.configs.CONFIGS["c4"].layers(False), dtype="f16", path="fused")
    src = m.kernel_source()
    assert "a_slots[kSlots * kSlotFrags * 64]" in src and "lds_vec" in src
    tab = src.split("chunk_tab[20] = {")[1].split("}")[0]
    assert [int(v) for v in tab.split(",")][1::2] == [32] * 10  # every c4 chunk is a full slot
    partial = create([P.Matvec(np.ones((40, 48))), P.Tanh(48), P.Matvec(np.ones((48, 80)))], dtype="f16",
                     path="fused").kernel_source()
    tab = partial.split("chunk_tab[")[1].split("{")[1].split("}")[0]
    assert [int(v) for v in tab.split(",")][1::2] == [6, 10]  # 3 tiles x 2 steps; 5 tiles x 2 steps
    deep = create(deep_half_chain(), dtype="f16", path="fused")
    src = deep.kernel_source()
    assert "lds_vec" not in src and "SeedRows{P + " in src
    deep.compile()


def test_input_in_contraction_order_only_for_contractions():
    """FUSED fp32 / fp64 plans whose input width is not a multiple of 16 load
    the input in contraction order, and skip the all-padding contraction
    steps, only when every read of the input state is a dense contraction
    (c5: two Dense layers and the projection skip)."""
    def src(layers, dtype="f32"):
        return create(layers, dtype=dtype, path="fused").kernel_source()

    c5 = src(P.configs.CONFIGS["c5"].layers(False))
    assert "load_rows_k<24>" in c5 and c5.count(", 6>(") == 3  # 24 inputs: 6 of 8 steps
    rng = np.random.default_rng(3)
    w = lambda a, b: rng.uniform(-0.3, 0.3, (a, b))  # noqa: E731
    assert "load_rows_k<24>" in src([P.Matvec(w(24, 32)), P.Relu(32)], "f64")
    assert "load_rows_k" not in src([P.Matvec(w(32, 32)), P.Relu(32)])  # no padding
    assert "load_rows_k" not in src([P.Relu(24), P.Matvec(w(24, 8))])  # pointwise on the input
    assert "load_rows_k" not in src([P.Save_State(0, 24), P.Matvec(w(24, 24)), P.Binop_Add(0, 24)])
    assert "load_rows_k" not in src([P.Save_State(0, 24), P.Matvec(w(24, 24)),
                                     P.Binop_Concatenate(0, 24, 48)])


def test_fused_config_sources():
    # c2's parameters sit in LDS: its dense epilogues are pinned among the
    # MFMAs (dense_ep_il); c3 streams its parameters from L2 and keeps dense_ep.
    for name in ["c2", "c3"]:
        m = create(P.configs.CONFIGS[name].layers(False))
        assert m.path == "fused"
        src = m.kernel_source()
        if name == "c2":
            assert src.count("dense_ep_il<16, ") == 4 and "dense_ep<" not in src
        else:
            assert src.count("dense_ep<") == 10 and "dense_ep_il<" not in src


def test_fused_occupancy_settled_by_compilation(tmp_path, monkeypatch):
    # The first compile measures register use: c3 spills at two waves per SIMD
    # and settles at one; c5 fits three.
    monkeypatch.setenv("PONNI_JIT_CACHE", str(tmp_path))
    monkeypatch.delenv("PONNI_FUSED_WAVES_PER_SIMD", raising=False)
    monkeypatch.delenv("PONNI_FUSED_WAVES", raising=False)
    want = {"c3": "__launch_bounds__(256, 1)", "c5": "__launch_bounds__(768, 3)"}
    for name, bounds in want.items():
        m = create(P.configs.CONFIGS[name].layers(False))
        m.compile()
        src = m.kernel_source()
        assert bounds in src, [l for l in src.splitlines() if "launch_bounds" in l]
