"""ctypes binding of libs2pamd.so (the MI355X verify path behind the C ABI of
include/s2pro/*.h).

Python here is plumbing for tests and benchmarks: device memory and streams
come from torch, every computation runs in the HIP kernels of the library.
Loading fails loudly when the library has not been built; there is no
fallback implementation.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("S2PAMD_LIB") or os.path.join(_HERE, "libs2pamd.so")

P = ctypes.c_void_p
I = ctypes.c_int
I64 = ctypes.c_int64
U64 = ctypes.c_uint64
F = ctypes.c_float
SZ = ctypes.c_size_t

S2P_VOCAB = 155776
S2P_HEAD_SLICE = 4097
WQ_INT4 = 0
WQ_INT8 = 1


class BackboneOpts(ctypes.Structure):
    _fields_ = [("n_layers", I), ("quant", I), ("head_quant", I), ("head_rows", I),
                ("max_rows", I), ("max_sessions", I), ("ctx_len", I), ("kv_bits", I)]


class RowPlan(ctypes.Structure):
    """Internal S2pRowPlan (csrc/prims_internal.h), used by stage-level tests;
    its size is checked against the library (s2p_test_desc_bytes)."""
    _fields_ = [("pos", P), ("slot", P), ("sess", P), ("vis", P), ("kv", P), ("kvs", P),
                ("layer_stride", I64), ("max_seq", I)]


class AttnSeg(ctypes.Structure):
    """Internal S2pAttnSeg (csrc/prims_internal.h)."""
    _fields_ = [("sess", ctypes.c_int32), ("L", ctypes.c_int32), ("row0", ctypes.c_int32),
                ("nrows", ctypes.c_int32), ("span", ctypes.c_int32), ("first", ctypes.c_int32),
                ("kv", P)]


class VerifyBatch(ctypes.Structure):
    _fields_ = [("n_sess", I), ("rows", I), ("parent", P), ("kv", P), ("kv_len", P),
                ("kv_scales", P)]


class StepIO(ctypes.Structure):
    _fields_ = [("x_in", P), ("logits", P), ("drf_logits", P), ("drf_stride", I64),
                ("parent_dev", P), ("tok_dev", P), ("states_dev", P), ("out_path", P),
                ("out_n_acc", P), ("out_emit", P), ("out_n_emit", P), ("work", P)]


class Tensor(ctypes.Structure):
    _fields_ = [("data", P), ("dtype", I), ("ndim", I), ("shape", I64 * 4), ("bytes", SZ),
                ("on_device", I)]


class Linear(ctypes.Structure):
    _fields_ = [("in_features", I), ("out_features", I), ("w_bf16", Tensor), ("w_fp8", Tensor),
                ("w_scales", Tensor), ("fp8_ready", I), ("w_int8", Tensor), ("w_iscale", Tensor),
                ("w_pack", Tensor), ("int8_ready", I), ("q_group", I), ("q_packed", I)]


class SlowLayer(ctypes.Structure):
    _fields_ = [("wqkv", Linear), ("wo", Linear), ("gate_up", Linear), ("w2", Linear),
                ("attn_norm", Tensor), ("ffn_norm", Tensor), ("q_norm", Tensor),
                ("k_norm", Tensor)]


class FaLayer(ctypes.Structure):
    """s2pfa_layer (include/s2pro/fastar.h)"""
    _fields_ = [("wqkv", Linear), ("wo", Linear), ("w13", Linear), ("w2", Linear),
                ("attn_norm", Tensor), ("ffn_norm", Tensor)]


class FaWeights(ctypes.Structure):
    """s2pfa_weights (include/s2pro/fastar.h)"""
    _fields_ = [("layers", FaLayer * 4), ("norm", Tensor), ("output", Linear),
                ("cb_emb", Tensor), ("emb", Tensor)]


class DraftModel(ctypes.Structure):
    """s2p_draft_model (include/s2pro/draft.h)"""
    _fields_ = [(n, Tensor) for n in
                ("fuse", "wqkv", "wo", "w1", "w3", "w2", "q_norm", "k_norm", "attn_norm",
                 "ffn_norm", "final_norm", "xcat", "x", "a", "qkv", "attn", "gu", "ffn")]


class DraftState(ctypes.Structure):
    """s2p_draft_state (include/s2pro/draft.h)"""
    _fields_ = [("kc", Tensor), ("vc", Tensor), ("pos", I)]


class SpecModel(ctypes.Structure):
    """s2p_spec_model (include/s2pro/spec.h)"""
    _fields_ = [("bb", P), ("draft", P), ("draft_states", P), ("fa", P), ("embed", P),
                ("n_sess", I), ("K", I)]


class SpecSessions(ctypes.Structure):
    """s2p_spec_sessions (include/s2pro/spec.h)"""
    _fields_ = [("kv", P), ("kv_len", P), ("prev_tok", P), ("prev_codes", P),
                ("prev_hidden", P), ("states", P), ("done", P)]


class SpecOut(ctypes.Structure):
    """s2p_spec_out (include/s2pro/spec.h)"""
    _fields_ = [("n_acc", P), ("n_emit", P), ("emit", P), ("frames", P)]


class SpecBuffers(ctypes.Structure):
    """s2p_spec_buffers (include/s2pro/spec.h)"""
    _fields_ = [("logits", P), ("drf_logits", P), ("x", P), ("tok", P), ("draft_codes", P),
                ("codes_out", P), ("path", P), ("tail", P), ("chain_ok", P), ("head_rows", I),
                ("replans", I)]


# name -> (restype, argtypes); every symbol declared in include/s2pro/*.h
SIGS = {
    # status.h / tensor.h
    "s2p_status_str": (ctypes.c_char_p, [I]),
    "s2p_dtype_size": (SZ, [I]),
    "s2p_tensor_numel": (I64, [P]),
    "s2p_tensor_device_alloc": (I, [P, I, I, P]),
    "s2p_tensor_free": (None, [P]),
    # gemm.h
    "s2p_gemm_init": (I, [I]),
    "s2p_gemm_shutdown": (None, []),
    "s2p_linear_from_device_bf16": (I, [P, P, I, I]),
    "s2p_linear_prepare_int8": (I, [P, P]),
    "s2p_linear_prepare_int8_site": (I, [P, I, P]),
    "s2p_linear_forward": (I, [P, P, P, I, I, P]),
    "s2p_linear_free": (None, [P]),
    "s2p_linear_init_random_int4": (I, [P, I, I, I, F, U64, P]),
    "s2p_linear_init_random_int8": (I, [P, I, I, F, U64, P]),
    "s2p_int8_quant": (I, [P, P, P, I, I, P]),
    "s2p_int8_gemv": (I, [P, P, P, P, I, I, I, P]),
    "s2p_int8_dequant": (I, [P, P, P, I, I, P]),
    "s2p_intq_quant": (I, [P, P, P, I, I, I, I, I, P]),
    "s2p_intq_gemv": (I, [P, P, P, P, I, I, I, I, P]),
    "s2p_intq_dequant": (I, [P, P, P, I, I, I, P]),
    "s2p_int4_pack": (I, [P, P, I, I, P]),
    "s2p_int4p_gemv": (I, [P, P, P, P, I, I, I, I, P]),
    "s2p_gemv_engine_run": (I, [I, I, P, P, P, P, I, I, I, P]),
    "s2p_int4p_gemm_tc_noalloc": (I, [P, P, P, P, I, I, I, I, P]),
    "s2p_int4p_gemm_tc": (I, [P, P, P, P, I, I, I, I, P]),
    "s2p_int4p_dequant": (I, [P, P, P, I, I, I, P]),
    "s2p_gemm_bf16": (I, [P, P, P, I, I, I, P]),
    # draft.h
    "s2p_draft_load": (I, [P, ctypes.c_char_p]),
    "s2p_draft_free": (None, [P]),
    "s2p_draft_state_init": (I, [P]),
    "s2p_draft_state_free": (None, [P]),
    "s2p_draft_step": (I, [P, P, P, P, P, P]),
    "s2p_draft_head": (I, [P, P, P, I, P]),
    "s2p_qcache_open": (I, [ctypes.c_char_p, I, P]),
    "s2p_qcache_reading": (I, [P]),
    "s2p_qcache_try_load": (I, [P, ctypes.c_char_p, I, I, P, P]),
    "s2p_qcache_put_linear": (I, [P, ctypes.c_char_p, P, P]),
    "s2p_qcache_finish": (I, [P, P]),
    "s2p_qcache_free": (None, [P]),
    # kernels.h
    "s2pk_rms_norm": (I, [P, P, P, I, I, F, P]),
    "s2pk_qk_norm": (I, [P, P, I, I, I, F, P]),
    "s2pk_rope": (I, [P, P, I, I, I, I, I, F, P]),
    "s2pk_kv_append": (I, [P, P, P, P, I, I, I, I, I, P]),
    "s2pk_attention": (I, [P, P, P, P, I, I, I, I, I, I, P]),
    "s2pk_silu_mul": (I, [P, P, I, I, P]),
    "s2pk_add": (I, [P, P, I64, P]),
    "s2pk_sample_prepare": (I, [P, P, I, P]),
    # slowar_kernels.h
    "s2pk_qkv_split": (I, [P, P, P, P, I, I, I, P]),
    "s2pk_rope_pos": (I, [P, P, I, I, I, I, P, F, P]),
    "s2pk_kv_append_ptrs": (I, [P, P, P, P, I, I, I, P, I, P]),
    "s2pk_attention_ptrs": (I, [P, P, P, P, I, I, I, I, P, I, P]),
    "s2pk_attention_decode": (I, [P, P, P, P, I, I, I, I, P, I, I, P, P]),
    "s2pk_attention_part_floats": (I64, [I, I, I]),
    "s2pk_kv_append8": (I, [P, P, P, P, P, P, I, I, I, I, I, I, P]),
    "s2pk_kv_append8_ptrs": (I, [P, P, P, P, P, P, I, I, I, P, I, I, P]),
    "s2pk_attention8": (I, [P, P, P, P, P, P, I, I, I, I, I, I, I, P]),
    "s2pk_attention8_decode": (I, [P, P, P, P, P, P, I, I, I, I, P, I, I, P, I, P]),
    "s2pk_sample": (I, [P, I64, P, P, I, P, P, P, P, P]),
    "s2pk_embed": (I, [P, P, P, I, I, P]),
    "s2pk_argmax": (I, [P, P, I, I, P]),
    # fastar.h
    "s2pfa_create": (I, [P, P, I, P]),
    "s2pfa_create_random": (I, [P, I, I, U64, P]),
    "s2pfa_free": (None, [P]),
    "s2pfa_weights_of": (ctypes.POINTER(FaWeights), [P]),
    "s2pfa_decode_frame_batch": (I, [P, P, P, I, P, P]),
    "s2pfa_decode_frame_batch_dev": (I, [P, P, P, I, P, P]),
    "s2pfa_decode_frame_logits_dev": (I, [P, P, P, I, P, P, P]),
    "s2pfa_vq_embed_add_dev": (I, [P, P, I, P, P]),
    "s2pfa_vq_embed_add": (I, [P, P, I, P, P]),
    # verify.h
    "s2p_backbone_create_random": (I, [P, U64, P, P]),
    "s2p_backbone_free": (None, [P]),
    "s2p_backbone_layer": (ctypes.POINTER(SlowLayer), [P, I]),
    "s2p_backbone_head": (ctypes.POINTER(Linear), [P]),
    "s2p_backbone_final_norm": (P, [P]),
    "s2p_backbone_kv_bytes": (SZ, [P]),
    "s2p_backbone_kv_scale_bytes": (SZ, [P]),
    "s2p_backbone_weight_bytes": (SZ, [P]),
    "s2p_verify_plan": (I, [P, P, P]),
    "s2p_verify_forward": (I, [P, P, P, P]),
    "s2p_verify_accept_work_bytes": (SZ, [I, I]),
    "s2p_verify_accept": (I, [P, P, P, P, I64, P, P, P, I, I, P, P, P, P, P, P]),
    "s2p_verify_kv_commit": (I, [P, P, P, P]),
    "s2p_verify_chain": (I, [P, P, P, P, P, P, P, P]),
    "s2p_verify_accept_chain": (I, [P, P, P, P, I64, P, P, P, I, I, P, P, P, P, P, P, P]),
    "s2p_verify_step": (I, [P, P, I, P]),
    "s2p_verify_status": (I, [P, P, I, P]),
    "s2p_verify_plan_device": (I, [P, P, P, P]),
    "s2p_spec_create": (I, [P, P, P, P, P, P]),
    "s2p_spec_tick": (I, [P, I, P]),
    "s2p_spec_buffers_of": (I, [P, P]),
    "s2p_spec_free": (None, [P]),
}

# synthetic-data launchers (csrc/synth_internal.h), used by tests/benchmarks
EXTRA = {
    "s2p_backbone_set_mk": (None, [P, I]),
    "s2p_test_f2bf": (I, [P, P, I64, P]),
    "s2p_test_desc_bytes": (SZ, [I]),
    "s2p_backbone_mk_status": (I, [P]),
    "s2p_backbone_set_mk_spin": (None, [P, ctypes.c_uint]),
    "s2p_synth_bytes": (I, [P, I64, U64, P]),
    "s2p_synth_int8": (I, [P, I64, U64, P]),
    "s2p_synth_f16_absnormal": (I, [P, I64, F, U64, P]),
    "s2p_synth_f32_absnormal": (I, [P, I64, F, U64, P]),
    "s2p_synth_bf16_normal": (I, [P, I64, F, F, U64, P]),
}

_lib = None


def load():
    """Load the built library (raises if it is missing)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built: run `make -C s2pro-native_amd` "
                "(or __graft_entry__.build()); there is no fallback path")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in {**SIGS, **EXTRA}.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc, what=""):
    if rc != 0:
        msg = load().s2p_status_str(rc)
        raise RuntimeError(f"{what}: s2p status {rc} ({msg.decode() if msg else '?'})")


def hip_check(rc, what=""):
    if rc != 0:
        raise RuntimeError(f"{what}: hipError {rc}")


def stream_ptr(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def dptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None
