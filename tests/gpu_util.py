"""Helpers of the GPU parity tests: device buffers (torch as plumbing), host
copies of raw device pointers, synthetic data."""
import ctypes

import numpy as np
import torch

import s2pamd

DEV = "cuda:0"
_hip = None
# Every device buffer made by to_dev()/empty() stays referenced until the test
# ends (conftest clears it after a device synchronisation): pointers handed to
# the C ABI must never outlive their torch tensor, whose block the caching
# allocator would otherwise hand to the next allocation.
LIVE = []
# (what, largest per-row gpu-oracle L2 distance, exception rows used, rows) of
# every logits check, summarised at the end of the pytest run (conftest)
LOGITS_RECORD = []


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
        t = torch.from_numpy(a.view(np.int16)).to(DEV)
    elif a.dtype == np.uint64:
        t = torch.from_numpy(a.view(np.int64)).to(DEV)
    else:
        t = torch.from_numpy(a).to(DEV)
    LIVE.append(t)
    return t


def to_host(t, dtype=None):
    sync()
    a = t.detach().cpu().numpy()
    if dtype is not None:
        a = a.view(dtype)
    return a


def empty(shape, dtype=torch.int16):
    t = torch.empty(shape, dtype=dtype, device=DEV)
    LIVE.append(t)
    return t


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


def assert_close_norm(got, want, rel=1e-2, what="", max_factor=2.0):
    """Per row: ||got - want||_2 <= rel ||want||_2 (the relative error of the
    row vector) and, as a guard against a few wild elements,
    max|got - want| <= max_factor * rel * max|want|; rel may be a per-row
    array."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    d = got - want
    l2 = np.linalg.norm(d, axis=-1) / np.maximum(np.linalg.norm(want, axis=-1), 1e-30)
    mx = np.abs(d).max(axis=-1) / np.maximum(np.abs(want).max(axis=-1), 1e-30)
    rel = np.broadcast_to(np.asarray(rel, np.float64), l2.shape)
    assert (l2 <= rel).all() and (mx <= max_factor * rel).all(), (
        f"{what}: worst row L2 rel {l2.max():.3g} (row {int(l2.argmax())}), "
        f"worst row max-norm rel {mx.max():.3g} (row {int(mx.argmax())}), "
        f"tolerance {rel.min():.3g}..{rel.max():.3g}; failing rows "
        f"{[(int(i), round(float(l2[i]), 4), round(float(mx[i]), 4), round(float(rel[i]), 4)) for i in np.nonzero((l2 > rel) | (mx > max_factor * rel))[0]]}")
