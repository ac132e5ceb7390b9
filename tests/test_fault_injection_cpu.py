"""The device-error contract, exercised without a GPU and without a GPU
fault: a host-only context of the C-ABI (MI355X_DEVICE_HOST_ONLY) and the
fault injection hook (mi355x_inject_fault, MI355X_INJECT_FAULT) make every
device entry point fail the way a HIP error would, and the ggml plugin must
turn that into GGML_STATUS_FAILED / false with an [mi355x error] message,
never a crash -- the reference's boundary contract (src/ggml-xdna.cpp:
299-305, 803-807: engine exceptions become false, then GGML_STATUS_FAILED)."""
import ctypes as C
import os
import subprocess
import sys
import textwrap

import pytest

import mi355x

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(os.path.dirname(HERE), "xdna.cpp_amd")


@pytest.fixture
def host_ctx():
    lib = mi355x.load()
    h = C.c_void_p()
    mi355x.check(lib.mi355x_ctx_create(mi355x.DEVICE_HOST_ONLY, C.byref(h)))
    yield lib, h
    mi355x.inject_fault(None)
    lib.mi355x_ctx_destroy(h)


def test_host_only_context_fails_every_device_call(host_ctx):
    lib, h = host_ctx
    assert lib.mi355x_ctx_device(h) == -1
    # options are host state
    mi355x.check(lib.mi355x_ctx_set_option(h, mi355x.OPT_VARIANT, mi355x.VARIANT_GGML_Q8))
    buf = (C.c_float * 64)()
    calls = {
        "mi355x_gemv": lambda: lib.mi355x_gemv(h, mi355x.Q4_0, buf, 32, 32, buf, buf),
        "mi355x_memcpy_h2d": lambda: lib.mi355x_memcpy_h2d(h, buf, buf, 16),
        "mi355x_memcpy_d2h": lambda: lib.mi355x_memcpy_d2h(h, buf, buf, 16),
        "mi355x_fill": lambda: lib.mi355x_fill(h, buf, 0, 16),
        "mi355x_ctx_sync": lambda: lib.mi355x_ctx_sync(h),
        "mi355x_ctx_fence": lambda: lib.mi355x_ctx_fence(h),
        "mi355x_malloc": lambda: lib.mi355x_malloc(h, 256, C.byref(C.c_void_p())),
        "mi355x_prepack_from_host": lambda: lib.mi355x_prepack_from_host(h, mi355x.Q4_0, 1, 32, buf, buf, 0, 18),
    }
    for name, call in calls.items():
        assert call() == mi355x.EHIP, name
        msg = mi355x.last_error()
        assert msg.startswith(name + ": hipErrorNoDevice") and "[host-only context]" in msg, msg
    # argument validation comes first: a bad shape is still EINVAL
    assert lib.mi355x_gemv(h, mi355x.Q4_0, buf, 32, 33, buf, buf) == mi355x.EINVAL
    assert "multiple of 32" in mi355x.last_error()
    # nothing to free on a host-only context, and no server on it
    mi355x.check(lib.mi355x_free(h, None))
    assert lib.mi355x_server_create(h, 2048, C.byref(C.c_void_p())) == mi355x.EHIP


def test_injected_fault_fires_once_after_skip(host_ctx):
    lib, h = host_ctx
    buf = (C.c_float * 64)()
    mi355x.inject_fault("mi355x_fill", mi355x.HIP_ERROR_ILLEGAL_ADDRESS, skip=1)
    assert lib.mi355x_fill(h, buf, 0, 16) == mi355x.EHIP
    assert "hipErrorNoDevice" in mi355x.last_error()             # skipped: the context's own error
    assert lib.mi355x_gemv(h, mi355x.Q4_0, buf, 32, 32, buf, buf) == mi355x.EHIP
    assert "hipErrorNoDevice" in mi355x.last_error()             # another entry point: not counted
    assert lib.mi355x_fill(h, buf, 0, 16) == mi355x.EHIP
    msg = mi355x.last_error()
    assert msg.startswith("mi355x_fill: hipErrorIllegalAddress") and msg.endswith("[injected]"), msg
    assert lib.mi355x_fill(h, buf, 0, 16) == mi355x.EHIP
    assert "hipErrorNoDevice" in mi355x.last_error()             # disarmed once fired


def test_injected_out_of_memory_and_any_entry(host_ctx):
    lib, h = host_ctx
    buf = (C.c_float * 64)()
    mi355x.inject_fault("*", mi355x.HIP_ERROR_OUT_OF_MEMORY)
    assert lib.mi355x_memcpy_d2h(h, buf, buf, 16) == mi355x.ENOMEM
    assert "hipErrorOutOfMemory" in mi355x.last_error() and "[injected]" in mi355x.last_error()
    # a fault on context creation (a device that fails to initialise)
    mi355x.inject_fault("mi355x_ctx_create", mi355x.HIP_ERROR_NO_DEVICE)
    out = C.c_void_p()
    assert lib.mi355x_ctx_create(0, C.byref(out)) == mi355x.EHIP and not out.value
    assert "[injected]" in mi355x.last_error()
    # bad arming arguments
    assert lib.mi355x_inject_fault(b"mi355x_gemv", 0, 0) == mi355x.EINVAL
    assert lib.mi355x_inject_fault(b"mi355x_gemv", 719, -1) == mi355x.EINVAL


# The plugin half runs in a child process: the host-only device is listed by
# the plugin's registry when MI355X_HOST_ONLY_DEVICE is set at its first use.
PLUGIN_SCRIPT = textwrap.dedent("""
    import ctypes as C, os, sys
    sys.path[:0] = [{tests!r}, {pkg!r}]
    import numpy as np
    import ggml_host as gh
    import mi355x
    lib = gh.bind_compat(mi355x.load())
    assert lib.ggml_backend_mi355x_set_op_mul_mat(gh.HOST_OP_MUL_MAT)
    reg = gh.Reg(lib.ggml_backend_init())
    n = reg.call("get_device_count")
    dev = reg.device(n - 1)
    assert dev.call("get_name") == b"MI355X_HOST_ONLY", dev.call("get_name")
    # a buffer cannot be allocated on it: NULL, not a crash
    bt = dev.buffer_type()
    assert not bt.call("alloc_buffer", 1 << 20)
    be = dev.backend()
    assert be is not None
    # a single-row Q4_0 MUL_MAT with host data (any address works: the
    # device gate fails before anything is read)
    K, N = 256, 64
    wmem = np.zeros(N * K // 32 * 18, np.uint8); xmem = np.ones(K, np.float32); ymem = np.zeros(N, np.float32)
    w = gh.tensor(gh.TYPE_Q4_0, [K, N], gh.contiguous_nb(18, 32, [K, N]), b"w"); w.data = wmem.ctypes.data
    x = gh.tensor(gh.TYPE_F32, [K, 1], gh.contiguous_nb(4, 1, [K, 1]), b"x"); x.data = xmem.ctypes.data
    o = gh.mul_mat(w, x, [N, 1], name=b"o"); o.data = ymem.ctypes.data
    o2 = gh.mul_mat(w, x, [N, 1], name=b"o2"); o2.data = ymem.ctypes.data
    print("graph_compute", be.compute([o]), flush=True)
    print("graph_compute_group", be.compute([o, o2]), flush=True)
    mi355x.inject_fault("mi355x_gemv", mi355x.HIP_ERROR_LAUNCH_FAILURE)
    print("graph_compute_injected", be.compute([o]), flush=True)
    # the compatibility entry point
    cw = gh.CompatTensor(type=gh.TYPE_Q4_0); cw.ne[:] = [K, N, 1, 1]; cw.data = wmem.ctypes.data
    cx = gh.CompatTensor(type=0); cx.ne[:] = [K, 1, 1, 1]; cx.data = xmem.ctypes.data
    co = gh.CompatTensor(type=0, op=gh.COMPAT_OP_MUL_MAT); co.ne[:] = [N, 1, 1, 1]; co.data = ymem.ctypes.data
    co.src[0] = C.addressof(cw); co.src[1] = C.addressof(cx)
    arr = (C.POINTER(gh.CompatTensor) * 1)(C.pointer(co))
    print("compute_graph", lib.ggml_backend_mi355x_compute_graph(be.addr, arr, 1), flush=True)
    # async copies and synchronize on a failing device: logged, no crash
    be.call("synchronize")
    be.free()
    print("done", flush=True)
""")


def test_plugin_turns_device_errors_into_failed_status():
    env = dict(os.environ, MI355X_HOST_ONLY_DEVICE="1")
    env.pop("MI355X_INJECT_FAULT", None)
    r = subprocess.run([sys.executable, "-c", PLUGIN_SCRIPT.format(tests=HERE, pkg=PKG)], env=env,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    out = dict((line.split(" ", 1) + [""])[:2] for line in r.stdout.splitlines())
    assert int(out["graph_compute"]) == -1          # GGML_STATUS_FAILED
    assert int(out["graph_compute_group"]) == -1
    assert int(out["graph_compute_injected"]) == -1
    assert out["compute_graph"] == "False"
    assert out["done"] == ""
    err = r.stderr
    assert "[mi355x error] node 'o' GEMV dispatch: mi355x_gemv: hipErrorNoDevice" in err, err
    assert "mi355x_gemv: hipErrorLaunchFailure" in err and "[injected]" in err, err
    assert "alloc_buffer" in err


def test_env_armed_fault_reaches_the_plugin():
    # MI355X_INJECT_FAULT arms the fault at the library's first use
    env = dict(os.environ, MI355X_HOST_ONLY_DEVICE="1", MI355X_INJECT_FAULT="mi355x_malloc:2")
    script = textwrap.dedent(f"""
        import sys
        sys.path[:0] = [{HERE!r}, {PKG!r}]
        import ggml_host as gh, mi355x
        lib = gh.bind_compat(mi355x.load())
        reg = gh.Reg(lib.ggml_backend_init())
        dev = reg.device(reg.call("get_device_count") - 1)
        print(bool(dev.buffer_type().call("alloc_buffer", 4096)))
    """)
    r = subprocess.run([sys.executable, "-c", script], env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "False", r.stdout + r.stderr
    assert "mi355x_malloc: hipErrorOutOfMemory" in r.stderr and "[injected]" in r.stderr, r.stderr
