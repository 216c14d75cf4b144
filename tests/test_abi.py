"""The C-ABI library (no GPU needed): it loads, exports every function the
public headers declare, and rejects bad arguments / lifecycle misuse before
touching the device, as the reference contract specifies (status codes of
include/s2pro/status.h; reference gemm.c:428 STATE before init,
int8_gemv.cu:840-845 INVALID shapes, kernels.h rows<=0 success)."""
import ctypes
import os
import re

import pytest

import s2pamd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HDR = os.path.join(ROOT, "include", "s2pro")
DECL = re.compile(r"^(?:const\s+)?[A-Za-z_][\w]*\s*\**\s+\**\s*(s2pk?_\w+)\s*\(", re.M)

S2P_OK, S2P_ERR_INVALID, S2P_ERR_STATE = 0, -1, -6


def declared():
    names = set()
    for f in sorted(os.listdir(HDR)):
        if f.endswith(".h"):
            src = open(os.path.join(HDR, f)).read()
            src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
            names.update(DECL.findall(src))
    return names


@pytest.fixture(scope="module")
def lib():
    return s2pamd.load()


def test_every_declared_symbol_is_exported(lib):
    names = declared()
    assert len(names) > 50, sorted(names)
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding covers the same set
    assert names <= set(s2pamd.SIGS), sorted(names - set(s2pamd.SIGS))


def test_status_strings(lib):
    lib.s2p_status_str.restype = ctypes.c_char_p
    assert lib.s2p_status_str(S2P_ERR_INVALID)
    assert lib.s2p_status_str(S2P_ERR_STATE)


def test_rows_zero_launchers_succeed_without_work(lib):
    assert lib.s2pk_rms_norm(None, None, None, 0, 2560, 1e-6, None) == 0
    assert lib.s2pk_qk_norm(None, None, 0, 32, 128, 1e-6, None) == 0
    assert lib.s2pk_silu_mul(None, None, 0, 9728, None) == 0
    assert lib.s2pk_attention(None, None, None, None, 0, 32, 8, 128, 0, 16, None) == 0


def test_argument_validation(lib):
    # acceptance: null buffers / zero sessions / too many rows
    args = [None] * 4 + [4097, None, None, None, 1, 5] + [None] * 4 + [None, None]
    assert lib.s2p_verify_accept(*args) == S2P_ERR_INVALID
    # verify entry points on a null backbone
    assert lib.s2p_verify_forward(None, None, None, None) == S2P_ERR_INVALID
    assert lib.s2p_verify_step(None, None, 0, None) == S2P_ERR_INVALID
    # the accept workspace size is a pure function
    assert lib.s2p_verify_accept_work_bytes(1, 5) > 0
    assert lib.s2p_verify_accept_work_bytes(8, 5) >= lib.s2p_verify_accept_work_bytes(1, 5)


def test_partial_sizes(lib):
    # split-K attention partials: rows x heads x splits x (128 + m, l)
    n1 = lib.s2pk_attention_part_floats(5, 32, 128)
    n2 = lib.s2pk_attention_part_floats(5, 32, 4096)
    assert n1 == 5 * 32 * 1 * 130
    assert n2 > n1 and n2 % (5 * 32 * 130) == 0


def test_internal_descriptor_mirrors_match(lib):
    """The ctypes mirrors of internal launch descriptors used by stage-level
    GPU tests have the library's sizes (a stale mirror would hand a kernel
    misread pointers)."""
    assert ctypes.sizeof(s2pamd.RowPlan) == lib.s2p_test_desc_bytes(0)
    assert ctypes.sizeof(s2pamd.AttnSeg) == lib.s2p_test_desc_bytes(1)
    names = ["BackboneOpts", "VerifyBatch", "StepIO", "Tensor", "Linear", "SlowLayer",
             "DraftModel", "DraftState"]
    for i, n in enumerate(names, start=2):
        assert ctypes.sizeof(getattr(s2pamd, n)) == lib.s2p_test_desc_bytes(i), n
