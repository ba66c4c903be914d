"""Helpers for the GPU parity tests: device buffers via torch, the decode
context, and reference conversions from library routines."""
import numpy as np

_ctx = None


def torch():
    import torch as T
    return T


def ctx():
    global _ctx
    if _ctx is None:
        import haagenti_amd as H
        _ctx = H.HipContext(0)
    return _ctx


def stream():
    return torch().cuda.current_stream().cuda_stream


def dev(a):
    T = torch()
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint64:
        t = T.from_numpy(a.view(np.int64)).cuda()
    elif a.dtype == np.uint32:
        t = T.from_numpy(a.view(np.int32)).cuda()
    elif a.dtype == np.uint16:
        t = T.from_numpy(a.view(np.int16)).cuda()
    else:
        t = T.from_numpy(a).cuda()
    return t


def empty_u8(n):
    return torch().zeros(max(int(n), 1), dtype=torch().uint8, device="cuda")


def sync():
    torch().cuda.synchronize()


def host_u8(t):
    return t.cpu().numpy().view(np.uint8)


def bf16_bits(f32):
    """Round-to-nearest-even bf16 bit patterns via torch's CPU conversion."""
    T = torch()
    return T.from_numpy(np.ascontiguousarray(f32, dtype=np.float32)).to(T.bfloat16) \
        .view(T.int16).numpy().view(np.uint16)


def f16_bits(f32):
    return np.ascontiguousarray(f32, dtype=np.float32).astype(np.float16).view(np.uint16)


def same_f32(a, b):
    """Bitwise equality, with any NaN equal to any NaN."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return bool((na == nb).all() and (a.view(np.uint32)[~na] == b.view(np.uint32)[~nb]).all())


_hip = None


def _hiprt():
    """The HIP runtime torch loaded (for raw-pointer copies in tests)."""
    global _hip
    if _hip is None:
        import ctypes
        torch()
        path = None
        with open("/proc/self/maps") as f:
            for ln in f:
                if "libamdhip64" in ln:
                    path = ln.split()[-1]
                    break
        _hip = ctypes.CDLL(path or "libamdhip64.so")
        _hip.hipMemcpy.restype = ctypes.c_int
        _hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    return _hip


def d2h(ptr, n):
    """n bytes at a raw device address, copied to the host (hipMemcpy)."""
    out = np.empty(int(n), np.uint8)
    assert _hiprt().hipMemcpy(out.ctypes.data, int(ptr), int(n), 2) == 0
    return out


def h2d(ptr, a):
    """Host bytes copied to a raw device address (hipMemcpy)."""
    a = np.ascontiguousarray(a, dtype=np.uint8)
    assert _hiprt().hipMemcpy(int(ptr), a.ctypes.data, a.size, 1) == 0
