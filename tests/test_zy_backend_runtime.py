"""The runtime calls the reference's MoE host makes of the driver, through the C ABI on the GPU: a kernel by
name from a gfx950 code object (cuModuleGetFunction), launched with a 3-D grid (the fast prefill's direct
cuLaunchKernel) and with LLB_LAUNCH's argument-address convention (a by-value struct, a float);
device-mapped host memory that kernels read and write in place (cuMemHostAlloc + cuMemHostGetDevicePointer);
an asynchronous host-to-device copy in stream order (cuMemcpyHtoDAsync). Argument checks run on the CPU."""
import ctypes as C
import os

import numpy as np
import pytest

import eureka_moe as em

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HSACO = os.path.join(ROOT, "eureka-engine_amd", "drv_kernels.hsaco")


class Span(C.Structure):  # DrvSpan (eureka-engine_amd/driver/drv_kernels.hip)
    _fields_ = [("src", C.c_uint64), ("dst", C.c_uint64), ("n", C.c_uint32), ("pad", C.c_uint32)]


def _args(*vals):
    arr = (C.c_void_p * len(vals))(*[C.cast(C.pointer(v), C.c_void_p) for v in vals])
    return arr, len(vals)


def test_launch_checks_answer_without_a_device():
    lib = em.load()
    args, n = _args(C.c_float(1.0))
    assert lib.llb_hip_launch3(None, 1, 1, 1, 64, 0, args, n) == -1
    assert lib.llb_hip_launch3(C.c_void_p(1), 1, 1, 0, 64, 0, args, n) == -1
    assert lib.llb_hip_launch3(C.c_void_p(1), 1, 1, 1, 2048, 0, args, n) == -1
    assert lib.llb_hip_launch3(C.c_void_p(1), 1, 1, 1, 64, 200 * 1024, args, n) == -1
    assert lib.llb_hip_launch3(C.c_void_p(1), 1, 1, 1, 64, 0, None, 2) == -1
    assert lib.llb_hip_host_alloc(16, None, None) == -1
    assert lib.llb_hip_copy_h2d_async(0, None, 16) == -1


@pytest.mark.gpu
def test_kernel_by_name_3d_grid_mapped_memory_and_async_copy(dev):
    lib = dev.lib
    mod, fn = C.c_uint64(), C.c_void_p()
    dev.check(lib.llb_hip_module_load(HSACO.encode(), C.byref(mod)))
    dev.check(lib.llb_hip_module_function(mod.value, b"llb_drv_stage", C.byref(fn)))
    n = 3000
    x = np.random.default_rng(1).standard_normal(n).astype(np.float32)
    # mapped host memory: the kernel reads it in place
    hp, hd = C.c_void_p(), C.c_uint64()
    dev.check(lib.llb_hip_host_alloc(n * 4, C.byref(hp), C.byref(hd)))
    hp2, hd2 = C.c_void_p(), C.c_uint64()
    dev.check(lib.llb_hip_host_alloc(n * 4, C.byref(hp2), C.byref(hd2)))
    try:
        C.memmove(hp.value, x.ctypes.data, n * 4)
        d1, d2 = dev.alloc(n * 4), dev.alloc(n * 4)
        # y = 0: mapped host -> device (times 2); y = 1: async-copied device buffer -> mapped host (times 2);
        # a z of 2 runs each block twice (the same stores)
        dev.check(lib.llb_hip_copy_h2d_async(d2, x.ctypes.data, n * 4))
        a, b, s = Span(hd.value, d1, n, 0), Span(d2, hd2.value, n, 0), C.c_float(2.0)
        args, na = _args(a, b, s)
        dev.check(lib.llb_hip_launch3(fn, (n + 255) // 256, 2, 2, 256, 0, args, na))
        dev.sync()
        assert np.array_equal(dev.read(d1, (n,), np.float32), 2 * x)
        back = np.frombuffer((C.c_float * n).from_address(hp2.value), np.float32)
        assert np.array_equal(back, 2 * x)
    finally:
        dev.check(lib.llb_hip_host_free(hp))
        dev.check(lib.llb_hip_host_free(hp2))
