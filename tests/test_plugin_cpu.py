"""ggml plugin surface that needs no device: the claim rule on the
compatibility tensor struct, the registry with zero devices, struct layouts.

Claim cases follow tests/test-backend.cpp:18-56 and
tests/test-kquants-gemv.cpp:360-409 of the reference, plus the remaining
branches of supports_op_impl (src/ggml-xdna.cpp:95-147)."""
import ctypes as C

import pytest

import ggml_host as gh
import mi355x

Q = {"Q4_0": 2, "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ3_XXS": 18, "IQ3_S": 21, "IQ2_S": 22,
     "IQ4_XS": 23}


@pytest.fixture(scope="module")
def plib():
    return gh.bind_compat(mi355x.load())


def compat_op(wtype, K, N, M=1, xtype=0, op=gh.COMPAT_OP_MUL_MAT):
    w = gh.CompatTensor(type=wtype)
    w.ne[:] = [K, N, 1, 1]
    x = gh.CompatTensor(type=xtype)
    x.ne[:] = [K, M, 1, 1]
    o = gh.CompatTensor(type=0, op=op)
    o.ne[:] = [N, M, 1, 1]
    o.src[0] = C.addressof(w)
    o.src[1] = C.addressof(x)
    return o, w, x


def claims(plib, o):
    return plib.ggml_backend_mi355x_supports_op(None, C.byref(o))


def claims_case(plib, *args):
    case = compat_op(*args)  # keeps the source tensors alive during the call
    return claims(plib, case[0])


def test_compat_claims_reference_q4_0_case(plib):
    # tests/test-backend.cpp:18-42: Q4_0 5120 x 17408 is claimed
    o, w, x = compat_op(Q["Q4_0"], 5120, 17408)
    assert claims(plib, o)
    # F32 weights fall back to the CPU (test-backend.cpp:45-49)
    w.type = 0
    assert not claims(plib, o)
    # RMS_NORM is not claimed (test-backend.cpp:52-55)
    norm = gh.CompatTensor(op=gh.COMPAT_OP_RMS_NORM)
    assert not claims(plib, norm)


@pytest.mark.parametrize("name", ["Q4_K", "Q5_K", "Q3_K", "Q6_K", "IQ4_XS", "IQ3_S"])
def test_compat_claims_kquants_decode_only(plib, name):
    # tests/test-kquants-gemv.cpp:369-406: 4096 x 5120 claimed for M=1,
    # rejected for M=8 and for K=5121
    o, w, x = compat_op(Q[name], 5120, 4096)
    assert claims(plib, o)
    x.ne[1] = 8
    assert not claims(plib, o)
    x.ne[1] = 1
    w.ne[0] = 5121
    assert not claims(plib, o)


def test_compat_block_alignment(plib):
    # Q4_0 needs K % 32, the 256-superblock types K % 256
    assert claims_case(plib, Q["Q4_0"], 32 * 3, 64)
    assert not claims_case(plib, Q["Q4_0"], 48, 64)
    assert claims_case(plib, Q["Q4_K"], 512, 64)
    assert not claims_case(plib, Q["Q4_K"], 288, 64)


def test_compat_size_cutoff(plib):
    # N >= 32 and N % 4 == 0 (src/ggml-xdna.cpp:111-112)
    assert claims_case(plib, Q["Q4_0"], 256, 32)
    assert not claims_case(plib, Q["Q4_0"], 256, 28)
    assert not claims_case(plib, Q["Q4_0"], 256, 34)
    assert claims_case(plib, Q["Q4_0"], 256, 36)


def test_compat_row_stride_and_activation_type(plib):
    o, w, x = compat_op(Q["Q4_0"], 256, 64)
    w.nb[1] = 8 * 18  # exact contiguous row bytes
    assert claims(plib, o)
    w.nb[1] = 8 * 18 + 2
    assert not claims(plib, o)
    w.nb[1] = 0
    x.type = 1  # F16 activations are not claimed
    assert not claims(plib, o)
    x.type = 0
    x.nb[0] = 8  # strided activation elements
    assert not claims(plib, o)


def test_compat_missing_sources_and_wrong_op(plib):
    o, w, x = compat_op(Q["Q4_0"], 256, 64)
    o.src[1] = None
    assert not claims(plib, o)
    o.src[1] = C.addressof(x)
    o.op = gh.COMPAT_OP_RMS_NORM
    assert not claims(plib, o)
    assert not plib.ggml_backend_mi355x_supports_op(None, None)


def test_compat_iq_grid_types_need_grids(plib):
    # IQ3_XXS / IQ2_S are claimed only once their ggml grids are installed
    for name in ("IQ3_XXS", "IQ2_S"):
        assert claims_case(plib, Q[name], 256, 64) == mi355x.type_ready(Q[name])


def test_compute_graph_rejects_bad_arguments(plib):
    assert not plib.ggml_backend_mi355x_compute_graph(None, None, 0)
    o, w, x = compat_op(Q["Q4_0"], 256, 64)
    arr = (C.POINTER(gh.CompatTensor) * 1)(C.pointer(o))
    assert not plib.ggml_backend_mi355x_compute_graph(None, arr, 1)
    assert plib.ggml_backend_mi355x_graph_compute(None, None) == gh.STATUS_FAILED
    assert not plib.ggml_backend_is_mi355x(None)


def test_registry_entry_points(plib):
    reg = gh.Reg(plib.ggml_backend_init())
    assert reg.api_version == 3
    assert reg.call("get_name") == b"MI355X"
    n = reg.call("get_device_count")
    assert n == mi355x.device_count()
    assert plib.ggml_backend_score() == (100 if n > 0 else 0)
    assert reg.device(n) is None
    for name in (b"ggml_backend_mi355x_init", b"ggml_backend_is_mi355x", b"ggml_backend_mi355x_free"):
        assert reg.call("get_proc_address", name)
    assert not reg.call("get_proc_address", b"no_such_function")
    assert plib.ggml_backend_mi355x_reg() == reg.addr
    if n == 0:
        assert plib.ggml_backend_mi355x_init(0) is None
        assert plib.ggml_backend_mi355x_buffer_type(0) is None


def test_set_op_mul_mat_validates(plib):
    assert not plib.ggml_backend_mi355x_set_op_mul_mat(-1)
    assert plib.ggml_backend_mi355x_set_op_mul_mat(gh.HOST_OP_MUL_MAT)


def test_iq_grid_loader_without_ggml_is_a_no_op(plib):
    # no ggml in this process: nothing to read the grids from
    assert plib.ggml_backend_mi355x_load_iq_grids_from_ggml() == 0


def test_struct_layouts():
    assert C.sizeof(gh.Tensor) == 336
    assert gh.Tensor.data.offset == 248 and gh.Tensor.op.offset == 80
    assert C.sizeof(gh.CompatTensor) == 304
    assert gh.CompatTensor.data.offset == 224


def test_compat_batch_broadcast_rule(plib):
    # weight batches must divide the activation batches (ggml's broadcast);
    # otherwise the weight index would run past the tensor
    o, w, x = compat_op(Q["Q4_0"], 2048, 256)
    for w2, x2, claimed in [(1, 1, True), (1, 4, True), (2, 4, True), (4, 4, True), (2, 3, False),
                            (3, 1, False), (4, 2, False)]:
        w.ne[2], x.ne[2], o.ne[2] = w2, x2, x2
        assert claims(plib, o) == claimed, (w2, x2)
    w.ne[2], x.ne[2], o.ne[2] = 1, 1, 1
    w.ne[3], x.ne[3], o.ne[3] = 2, 3, 3
    assert not claims(plib, o)
    w.ne[3], x.ne[3], o.ne[3] = 1, 2, 1  # output batches must be the activation batches
    assert not claims(plib, o)
