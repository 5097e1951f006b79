"""numpy/ctypes front end of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, to check results against.  The product (channel_amd/)
never imports it.  Every function restates reference semantics; see
oracle.c for the file:line each one follows.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u32, _u64, _f32, _int, _size = (ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float,
                                 ctypes.c_int, ctypes.c_size_t)

_PROTOS = {
    "orc_f32_to_f16": (ctypes.c_uint16, [_f32]),
    "orc_f16_to_f32": (_f32, [ctypes.c_uint16]),
    "orc_bf16_from_f32": (ctypes.c_uint16, [_f32]),
    "orc_bf16_to_f32": (_f32, [ctypes.c_uint16]),
    "orc_quantize_matrix_q4": (None, [_u32p, _u16p, _size, _size]),
    "orc_quantize_matrix_q8": (None, [_u32p, _u16p, _size, _size]),
    "orc_dequant_q4": (None, [_f32p, _u32p, _size, _size]),
    "orc_dequant_q8": (None, [_f32p, _u32p, _size, _size]),
    "orc_gelu_tanh": (_f32, [_f32]),
    "orc_gemv_q4": (None, [_u32p, _f32p, _f32p, _u32, _u32]),
    "orc_fused_qkv_q4": (None, [_u32p, _u32p, _u32p, _f32p, _f32p, _f32p, _f32p, _u32, _u32, _u32]),
    "orc_fused_mlp_q4": (None, [_u32p, _u32p, _f32p, _f32p, _u32, _u32]),
    "orc_gemv_q8": (None, [_u32p, _f32p, _f32p, _u32, _u32]),
    "orc_batch_gemm_q4": (None, [_u32p, _f32p, _f32p, _u32, _u32, _u32]),
    "orc_batch_fused_mlp_q4": (None, [_u32p, _u32p, _f32p, _f32p, _u32, _u32, _u32]),
    "orc_batch_gemm_q4_bf16": (None, [_u32p, _f32p, _f32p, _u32, _u32, _u32]),
    "orc_decode_attn": (None, [_f32p, _f32p, _f32p, _u32p, _u32, _u32, _u32, _u32, _u32, _f32,
                               _f32p]),
    "orc_qkv_rope": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _u32, _u32,
                            _u32, _u32, _int, _f32, _f32, _u32, _u32]),
    "orc_rmsnorm": (None, [_f32p, _f32p, _f32p, _u32, _f32]),
    "orc_add_rmsnorm": (None, [_f32p, _f32p, _f32p, _f32p, _u32, _f32, _f32]),
    "orc_batch_causal_attn": (None, [_f32p, _f32p, _f32p, _u32p, _u32, _u32, _u32, _u32, _u32,
                                     _u32, _f32, _u32, _f32p]),
    "orc_softcap": (_f32, [_f32]),
    "orc_topk64": (None, [_f32p, _u32, _u32p, _f32p]),
    "orc_argmax": (_u32, [_f32p, _u32]),
    "orc_mix64": (_u64, [_u64, _u64]),
    "orc_synth_q4": (None, [_u32p, _u32, _u32, _u64, _f32, _f32]),
    "orc_synth_q8": (None, [_u32p, _u32, _u32, _u64, _f32, _f32]),
    "orc_synth_normal": (None, [_f32p, _size, _u64, _f32]),
    "orc_gemv_q4_mt": (None, [_u32p, _f32p, _f32p, _u32, _u32, _int]),
    "orc_fused_mlp_step_mt": (None, [_u32p, _u32p, _u32p, _f32p, _f32p, _f32p, _u32, _u32, _int]),
    "orc_gemv_q8_mt": (None, [_u32p, _f32p, _f32p, _u32, _u32, _int]),
    "orc_quantize_matrix_q4_mt": (None, [_u32p, _u16p, _size, _size, _int]),
    "orc_quantize_matrix_q8_mt": (None, [_u32p, _u16p, _size, _size, _int]),
    "orc_batch_gemm_q4_bf16_mt": (None, [_u32p, _f32p, _f32p, _u32, _u32, _u32, _int]),
    "orc_fused_mlp_q4_mt": (None, [_u32p, _u32p, _f32p, _f32p, _u32, _u32, _int]),
    "orc_batch_causal_attn_mt": (None, [_f32p, _f32p, _f32p, _u32p, _u32, _u32, _u32, _u32, _u32,
                                        _u32, _f32, _u32, _f32p, _int]),
    "orc_gelu_tanh_vec": (None, [_f32p, _f32p, _size]),
    "orc_quiescence_gate": (_int, [_f32p, _f32p, _u32, _f32, _f32p]),
    "orc_softcap_vec": (None, [_f32p, _f32p, _size]),
}

# Threads for the checking forms at full model sizes (results are
# bit-identical to the serial routines whatever the count).
NTHREADS = max(1, min(16, len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()))


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built (make -C oracle)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in _PROTOS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def _c(a, dtype, need=None):
    """Contiguous array of dtype; with `need`, at least that many elements
    (the C routines read exactly the sizes their arguments imply)."""
    out = np.ascontiguousarray(a, dtype=dtype)
    if need is not None and out.size < need:
        raise ValueError(f"buffer of {out.size} elements, need {need}")
    return out


def _q4(W, rows, K):
    return _c(W, np.uint32, rows * (K // 32) * 5)


def _q8(W, rows, K):
    return _c(W, np.uint32, rows * (K // 32) * 9)


def f32_to_f16_bits(v):
    return np.array([lib.orc_f32_to_f16(float(x)) for x in np.ravel(v)], dtype=np.uint16)


def f16_bits_to_f32(h):
    return np.array([lib.orc_f16_to_f32(int(x)) for x in np.ravel(h)], dtype=np.float32)


def bf16_from_f32(v):
    return np.array([lib.orc_bf16_from_f32(float(x)) for x in np.ravel(v)], dtype=np.uint16)


def quantize_q4(w_bf16, nthreads=1):
    """[rows, cols] bf16 bits -> Q4 words [rows, cols/32*5] (quant.zig:58-98)."""
    w = _c(w_bf16, np.uint16)
    rows, cols = w.shape
    out = np.zeros((rows, (cols + 31) // 32 * 5), dtype=np.uint32)
    if nthreads > 1:
        lib.orc_quantize_matrix_q4_mt(out, w, rows, cols, int(nthreads))
    else:
        lib.orc_quantize_matrix_q4(out, w, rows, cols)
    return out


def quantize_q8(w_bf16, nthreads=1):
    w = _c(w_bf16, np.uint16)
    rows, cols = w.shape
    out = np.zeros((rows, (cols + 31) // 32 * 9), dtype=np.uint32)
    if nthreads > 1:
        lib.orc_quantize_matrix_q8_mt(out, w, rows, cols, int(nthreads))
    else:
        lib.orc_quantize_matrix_q8(out, w, rows, cols)
    return out


def dequant_q4(W, rows, K):
    out = np.zeros((rows, K), dtype=np.float32)
    lib.orc_dequant_q4(out, _q4(W, rows, K), rows, K)
    return out


def dequant_q8(W, rows, K):
    out = np.zeros((rows, K), dtype=np.float32)
    lib.orc_dequant_q8(out, _q8(W, rows, K), rows, K)
    return out


def gelu_tanh(x):
    a = _c(np.ravel(x), np.float32)
    y = np.zeros(a.size, np.float32)
    lib.orc_gelu_tanh_vec(a, y, a.size)
    return y


def gemv_q4(W, x, M, K, nthreads=1):
    y = np.zeros(M, dtype=np.float32)
    if nthreads > 1:
        lib.orc_gemv_q4_mt(_q4(W, M, K), _c(x, np.float32, K), y, M, K, int(nthreads) - 1)
    else:
        lib.orc_gemv_q4(_q4(W, M, K), _c(x, np.float32, K), y, M, K)
    return y


def gemv_q4_mt(W, x, M, K, nthreads):
    y = np.zeros(M, dtype=np.float32)
    lib.orc_gemv_q4_mt(_q4(W, M, K), _c(x, np.float32, K), y, M, K, int(nthreads))
    return y


def fused_qkv_q4(Wq, Wk, Wv, x, q_dim, kv_dim, K, nthreads=1):
    if nthreads > 1:
        return (gemv_q4(Wq, x, q_dim, K, nthreads), gemv_q4(Wk, x, kv_dim, K, nthreads),
                gemv_q4(Wv, x, kv_dim, K, nthreads))
    q = np.zeros(q_dim, np.float32)
    k = np.zeros(kv_dim, np.float32)
    v = np.zeros(kv_dim, np.float32)
    lib.orc_fused_qkv_q4(_c(Wq, np.uint32), _c(Wk, np.uint32), _c(Wv, np.uint32),
                         _c(x, np.float32), q, k, v, q_dim, kv_dim, K)
    return q, k, v


def fused_mlp_q4(Wg, Wu, x, M, K, nthreads=1):
    act = np.zeros(M, np.float32)
    if nthreads > 1:
        lib.orc_fused_mlp_q4_mt(_q4(Wg, M, K), _q4(Wu, M, K), _c(x, np.float32, K), act, M, K, int(nthreads))
    else:
        lib.orc_fused_mlp_q4(_q4(Wg, M, K), _q4(Wu, M, K), _c(x, np.float32, K), act, M, K)
    return act


def fused_mlp_step_mt(Wg, Wu, Wd, x, H, I, nthreads):
    act = np.zeros(I, np.float32)
    y = np.zeros(H, np.float32)
    lib.orc_fused_mlp_step_mt(_c(Wg, np.uint32), _c(Wu, np.uint32), _c(Wd, np.uint32),
                              _c(x, np.float32), act, y, H, I, int(nthreads))
    return act, y


def gemv_q8_mt(W, x, M, K, nthreads):
    y = np.zeros(M, dtype=np.float32)
    lib.orc_gemv_q8_mt(_q8(W, M, K), _c(x, np.float32, K), y, M, K, int(nthreads))
    return y


def gemv_q8(W, x, M, K, nthreads=1):
    y = np.zeros(M, dtype=np.float32)
    if nthreads > 1:
        lib.orc_gemv_q8_mt(_q8(W, M, K), _c(x, np.float32, K), y, M, K, int(nthreads) - 1)
    else:
        lib.orc_gemv_q8(_q8(W, M, K), _c(x, np.float32, K), y, M, K)
    return y


def batch_gemm_q4(W, X, n_tok, M, K):
    Y = np.zeros((n_tok, M), np.float32)
    lib.orc_batch_gemm_q4(_q4(W, M, K), _c(X, np.float32, n_tok * K), Y, n_tok, M, K)
    return Y


def batch_gemm_q4_bf16(W, X, n_tok, M, K, nthreads=1):
    Y = np.zeros((n_tok, M), np.float32)
    if nthreads > 1:
        lib.orc_batch_gemm_q4_bf16_mt(_q4(W, M, K), _c(X, np.float32, n_tok * K), Y, n_tok, M, K, int(nthreads))
    else:
        lib.orc_batch_gemm_q4_bf16(_q4(W, M, K), _c(X, np.float32, n_tok * K), Y, n_tok, M, K)
    return Y


def batch_fused_mlp_q4(Wg, Wu, X, n_tok, M, K):
    Y = np.zeros((n_tok, M), np.float32)
    lib.orc_batch_fused_mlp_q4(_c(Wg, np.uint32), _c(Wu, np.uint32), _c(X, np.float32), Y,
                               n_tok, M, K)
    return Y


def decode_attn(Q, Kc, Vc, slots, num_q_heads, head_dim, kv_dim, gqa, scale=1.0):
    out = np.zeros(num_q_heads * head_dim, np.float32)
    s = _c(slots, np.uint32)
    lib.orc_decode_attn(_c(Q, np.float32), _c(Kc, np.float32), _c(Vc, np.float32), s, len(s),
                        num_q_heads, head_dim, kv_dim, gqa, scale, out)
    return out


def batch_causal_attn(Q, Kc, Vc, slots, n_tok, num_prev, num_q_heads, head_dim, kv_dim, gqa,
                      scale=1.0, window=0, nthreads=1):
    out = np.zeros(n_tok * num_q_heads * head_dim, np.float32)
    args = (_c(Q, np.float32), _c(Kc, np.float32), _c(Vc, np.float32), _c(slots, np.uint32), n_tok, num_prev,
            num_q_heads, head_dim, kv_dim, gqa, scale, window, out)
    if nthreads > 1:
        lib.orc_batch_causal_attn_mt(*args, int(nthreads))
    else:
        lib.orc_batch_causal_attn(*args)
    return out


def qkv_rope(q_in, k_in, v_in, q_norm_w, k_norm_w, k_cache, v_cache, num_q_heads, num_kv_heads,
             head_dim, rotary_dim, k_eq_v, theta, eps, clock, slot_idx):
    """Returns q_out; k_cache / v_cache (float32, C-contiguous) are updated in place."""
    q_out = np.zeros(num_q_heads * head_dim, np.float32)
    assert k_cache.dtype == np.float32 and k_cache.flags.c_contiguous
    assert v_cache.dtype == np.float32 and v_cache.flags.c_contiguous
    lib.orc_qkv_rope(_c(q_in, np.float32), _c(k_in, np.float32), _c(v_in, np.float32),
                     _c(q_norm_w, np.float32), _c(k_norm_w, np.float32), q_out, k_cache, v_cache,
                     num_q_heads, num_kv_heads, head_dim, rotary_dim, int(k_eq_v), theta, eps,
                     clock, slot_idx)
    return q_out


def rmsnorm(x, w, eps):
    y = np.zeros(len(x), np.float32)
    lib.orc_rmsnorm(_c(x, np.float32), _c(w, np.float32), y, len(x), eps)
    return y


def add_rmsnorm(x, r, w, eps, scalar):
    """Returns (x_updated, y)."""
    xx = np.array(x, dtype=np.float32, copy=True)
    y = np.zeros(len(xx), np.float32)
    lib.orc_add_rmsnorm(xx, _c(r, np.float32), _c(w, np.float32), y, len(xx), eps, scalar)
    return xx, y


def softcap(v):
    a = _c(np.ravel(v), np.float32)
    y = np.zeros(a.size, np.float32)
    lib.orc_softcap_vec(a, y, a.size)
    return y


def topk64(logits):
    ids = np.zeros(64, np.uint32)
    vals = np.zeros(64, np.float32)
    lg = _c(logits, np.float32)
    lib.orc_topk64(lg, len(lg), ids, vals)
    return ids, vals


def argmax(v):
    a = _c(v, np.float32)
    return int(lib.orc_argmax(a, len(a)))


def mix64(seed, idx):
    return int(lib.orc_mix64(seed, idx))


def synth_q4(rows, K, seed, smin=0.005, smax=0.02):
    W = np.zeros(rows * (K // 32) * 5, np.uint32)
    lib.orc_synth_q4(W, rows, K, seed, smin, smax)
    return W


def synth_q8(rows, K, seed, smin, smax):
    W = np.zeros(rows * (K // 32) * 9, np.uint32)
    lib.orc_synth_q8(W, rows, K, seed, smin, smax)
    return W


def synth_normal(n, seed, stddev=1.0):
    out = np.zeros(n, np.float32)
    lib.orc_synth_normal(out, n, seed, stddev)
    return out


def quiescence_gate(x, x_prev, thresh):
    """shaders/quiescence_gate.wgsl for one layer: returns (runs, mean
    square of the change); x_prev (float32, C-contiguous) is overwritten with x."""
    assert x_prev.dtype == np.float32 and x_prev.flags.c_contiguous
    xx = _c(x, np.float32, x_prev.size)
    ms = np.zeros(1, np.float32)
    runs = bool(lib.orc_quiescence_gate(xx, x_prev, x_prev.size, float(thresh), ms))
    return runs, float(ms[0])
