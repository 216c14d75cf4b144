"""Helpers of the GPU parity tests: device buffers (torch as plumbing), host
copies of raw device pointers, synthetic data."""
import ctypes

import numpy as np
import torch

import s2pamd

DEV = "cuda:0"
_hip = None


def hip():
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipMemcpy.restype = ctypes.c_int
        _hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        _hip.hipDeviceSynchronize.restype = ctypes.c_int
    return _hip


def sync():
    torch.cuda.synchronize()


def d2h(ptr, nbytes, dtype):
    """Copy nbytes from a raw device pointer into a new numpy array."""
    sync()
    out = np.empty(nbytes // np.dtype(dtype).itemsize, dtype)
    rc = hip().hipMemcpy(out.ctypes.data, ptr, nbytes, 2)
    assert rc == 0, f"hipMemcpy D2H failed: {rc}"
    return out


def h2d_raw(host, dev_ptr):
    """Copy a numpy array into raw device memory."""
    host = np.ascontiguousarray(host)
    rc = hip().hipMemcpy(dev_ptr, host.ctypes.data, host.nbytes, 1)
    assert rc == 0, f"hipMemcpy H2D failed: {rc}"
    sync()


def to_dev(a):
    """numpy -> device tensor (uint16 travels as int16 bits)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).to(DEV)
    if a.dtype == np.uint8:
        return torch.from_numpy(a).to(DEV)
    if a.dtype == np.uint64:
        return torch.from_numpy(a.view(np.int64)).to(DEV)
    return torch.from_numpy(a).to(DEV)


def to_host(t, dtype=None):
    sync()
    a = t.detach().cpu().numpy()
    if dtype is not None:
        a = a.view(dtype)
    return a


def empty(shape, dtype=torch.int16):
    return torch.empty(shape, dtype=dtype, device=DEV)


def P(t):
    return s2pamd.dptr(t)


def S():
    return s2pamd.stream_ptr()


def bf16_bits(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).view(
        torch.int16).numpy().view(np.uint16)


def bf16_vals(bits):
    return (np.ascontiguousarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def assert_close_rel(got, want, rel=1e-2, floor_frac=1e-2, what=""):
    """|got - want| <= rel * |want| + floor_frac * rms(want), elementwise."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    rms = float(np.sqrt(np.mean(want ** 2))) if want.size else 0.0
    err = np.abs(got - want)
    bound = rel * np.abs(want) + floor_frac * rms
    bad = err > bound
    assert not bad.any(), (
        f"{what}: {int(bad.sum())}/{bad.size} beyond tolerance; max err {err.max():.4g} "
        f"(rms {rms:.4g}); worst at {np.unravel_index(np.argmax(err - bound), err.shape)}")
