"""ctypes binding of include/channel_hip.h (libchannel_hip.so).

The library is the product: every compute call goes to hand-written gfx950
HIP kernels behind the C-ABI.  There is no fallback; if the shared library is
missing, importing this module raises.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libchannel_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "channel_hip.h")

c_void_p = ctypes.c_void_p
c_u32 = ctypes.c_uint32
c_u64 = ctypes.c_uint64
c_int = ctypes.c_int
c_f32 = ctypes.c_float
c_size = ctypes.c_size_t
P = ctypes.POINTER

STATUS_NAMES = {
    0: "OK",
    -1: "Invalid",
    -2: "HipError",
    -3: "NoDevice",
    -4: "OutOfMemory",
    -5: "BatchTooLarge",
    -6: "Unsupported",
}

# name -> (restype, argtypes)
PROTOTYPES = {
    "chn_device_count": (c_int, [P(c_int)]),
    "chn_init": (c_int, [c_int, P(c_void_p)]),
    "chn_destroy": (None, [c_void_p]),
    "chn_last_error": (ctypes.c_char_p, [c_void_p]),
    "chn_device_name": (ctypes.c_char_p, [c_void_p]),
    "chn_alloc": (c_int, [c_void_p, c_size, P(c_void_p)]),
    "chn_free": (c_int, [c_void_p, c_void_p]),
    "chn_upload": (c_int, [c_void_p, c_void_p, c_void_p, c_size]),
    "chn_download": (c_int, [c_void_p, c_void_p, c_void_p, c_size]),
    "chn_copy": (c_int, [c_void_p, c_void_p, c_void_p, c_size]),
    "chn_fill_u32": (c_int, [c_void_p, c_void_p, c_u32, c_size]),
    "chn_sync": (c_int, [c_void_p]),
    "chn_timer_start": (c_int, [c_void_p]),
    "chn_timer_stop": (c_int, [c_void_p, P(c_f32)]),
    "chn_record_begin": (c_int, [c_void_p]),
    "chn_record_end": (c_int, [c_void_p, P(c_void_p)]),
    "chn_submit": (c_int, [c_void_p, c_void_p]),
    "chn_recording_free": (None, [c_void_p]),
    "chn_gemv_q4": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_u32, c_u32]),
    "chn_fused_qkv_q4": (c_int, [c_void_p] + [c_void_p] * 7 + [c_u32, c_u32, c_u32]),
    "chn_fused_mlp_q4": (c_int, [c_void_p] + [c_void_p] * 4 + [c_u32, c_u32]),
    "chn_q4_repack": (c_int, [c_void_p, c_void_p, c_u32, c_u32, c_void_p]),
    "chn_gemv_q4r": (c_int, [c_void_p] * 4 + [c_u32, c_u32]),
    "chn_fused_qkv_q4r": (c_int, [c_void_p] * 8 + [c_u32, c_u32, c_u32]),
    "chn_fused_mlp_q4r": (c_int, [c_void_p] * 5 + [c_u32, c_u32]),
    "chn_xplanes": (c_int, [c_void_p, c_void_p, c_u32, c_void_p]),
    "chn_gemv_q4r_xp": (c_int, [c_void_p] * 4 + [c_u32, c_u32]),
    "chn_fused_mlp_q4r_xp": (c_int, [c_void_p] * 6 + [c_u32, c_u32]),
    "chn_ffn_gate_up_q4r": (c_int, [c_void_p] * 11 + [c_u32, c_u32, c_f32]),
    "chn_batch_gemm_q4": (c_int, [c_void_p] * 4 + [c_u32] * 3),
    "chn_batch_fused_mlp_q4": (c_int, [c_void_p] * 5 + [c_u32] * 3),
    "chn_batch_gemm_q4r": (c_int, [c_void_p] * 4 + [c_u32] * 3),
    "chn_batch_qkv_q4r": (c_int, [c_void_p] * 8 + [c_u32] * 4),
    "chn_batch_fused_mlp_q4r": (c_int, [c_void_p] * 6 + [c_u32] * 3),
    "chn_qkv_rope": (c_int, [c_void_p] + [c_void_p] * 9 + [c_u32] * 4 + [c_int, c_f32, c_f32]),
    "chn_decode_attn": (c_int, [c_void_p] + [c_void_p] * 5 + [c_u32] * 5 + [c_f32, c_void_p]),
    "chn_decode_attn_noalloc": (c_int, [c_void_p] + [c_void_p] * 5 + [c_u32] * 5 + [c_f32, c_void_p]),
    "chn_rmsnorm": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_u32, c_f32]),
    "chn_add_rmsnorm": (c_int, [c_void_p] * 5 + [c_u32, c_f32, c_f32]),
    "chn_batch_rmsnorm": (c_int, [c_void_p] * 4 + [c_u32, c_u32, c_f32]),
    "chn_batch_add_rmsnorm": (c_int, [c_void_p] * 5 + [c_u32, c_u32, c_f32, c_f32]),
    "chn_batch_qkv_rope": (c_int, [c_void_p] + [c_void_p] * 9 + [c_u32] * 7 + [c_int, c_f32, c_f32]),
    "chn_batch_causal_attn": (c_int, [c_void_p] * 5 + [c_u32] * 6 + [c_f32, c_u32, c_void_p]),
    "chn_gemv_q8": (c_int, [c_void_p] * 4 + [c_u32, c_u32]),
    "chn_q8_repack": (c_int, [c_void_p, c_void_p, c_u32, c_u32, c_void_p]),
    "chn_gemv_q8r": (c_int, [c_void_p] * 4 + [c_u32, c_u32]),
    "chn_topk64": (c_int, [c_void_p, c_void_p, c_u32, c_void_p, c_void_p]),
    "chn_quantize_q4": (c_int, [c_void_p] * 3 + [c_u32, c_u32]),
    "chn_quantize_q8": (c_int, [c_void_p] * 3 + [c_u32, c_u32]),
    "chn_to_bf16_bits": (c_int, [c_void_p] * 3 + [c_size]),
    "chn_model_create": (c_int, [c_void_p] * 5 + [P(c_void_p)]),
    "chn_model_create_synthetic": (c_int, [c_void_p, c_void_p, c_u64, P(c_void_p)]),
    "chn_model_destroy": (None, [c_void_p]),
    "chn_model_get_config": (c_int, [c_void_p, c_void_p]),
    "chn_model_embedding_bf16": (c_int, [c_void_p, P(c_void_p)]),
    "chn_model_set_graph": (c_int, [c_void_p, c_int]),
    "chn_decode_step": (c_int, [c_void_p, c_void_p, c_u32, c_u32, c_void_p, c_u32, c_void_p, c_u32,
                                c_void_p, c_void_p, P(c_u32)]),
    "chn_decode_token": (c_int, [c_void_p, c_u32, c_u32, c_u32, c_void_p, c_u32, c_void_p, c_u32,
                                 c_void_p, c_void_p, P(c_u32)]),
    "chn_decode_greedy": (c_int, [c_void_p, c_u32, c_u32, c_u32, c_void_p, c_void_p]),
    "chn_prefill": (c_int, [c_void_p, c_void_p, c_u32, c_void_p, c_void_p, c_u32, c_u32, c_u32,
                            c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "chn_kv_read": (c_int, [c_void_p, c_u32, c_u32, c_u32, c_void_p, c_void_p]),
    "chn_kv_write": (c_int, [c_void_p, c_u32, c_u32, c_u32, c_void_p, c_void_p]),
    "chn_model_read_state": (c_int, [c_void_p, c_void_p, c_void_p]),
    "chn_model_read_logits": (c_int, [c_void_p, c_void_p]),
    "chn_model_replay": (c_int, [c_void_p, c_int, c_void_p, c_void_p]),
    "chn_synth_q4": (c_int, [c_void_p, c_void_p, c_u32, c_u32, c_u64, c_f32, c_f32]),
    "chn_synth_q8": (c_int, [c_void_p, c_void_p, c_u32, c_u32, c_u64, c_f32, c_f32]),
    "chn_synth_normal": (c_int, [c_void_p, c_void_p, c_size, c_u64, c_f32]),
}


class ChannelError(RuntimeError):
    """A negative status from the C-ABI, with chn_last_error()'s text."""

    def __init__(self, fn, code, msg):
        self.code = code
        self.status = STATUS_NAMES.get(code, str(code))
        super().__init__(f"{fn} -> {self.status} ({code}): {msg}")


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()
