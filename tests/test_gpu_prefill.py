"""GPU parity of the MFMA prefill contractions (batch_gemm_q4,
batch_fused_mlp_q4).  Two references: the oracle's bf16-operand model (same
operand roundings as the MFMA path; only fp32 summation order differs, so
the bar is 1e-4) and the reference's fp32 semantics (the stated bar for
bf16-MFMA prefill, 1e-2).  Large shapes are checked on a token subset, full
width."""
import numpy as np
import pytest

import oracle
from gpu_util import f32_host, q4_host, rel_err, say, synth_normal_dev, synth_q4_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n_tok,M,K,sample", [
    (512, 15360, 3840, 12),    # config: prefill Q4 GEMM 512 x 3840 -> 15360 (128 x 128 tiles)
    (300, 16400, 64, None),    # 128 x 128 tiles, ragged tokens and features, one K step
    (512, 3840, 15360, 6),     # down_proj shape (128 x 128 tiles, K split in two)
    (512, 2048, 3840, 6),      # k/v shape (128 x 64 tiles, K split in two)
    (100, 200, 96, None),      # ragged: tokens, features and K not tile multiples
    (1, 130, 32, None),        # one token, one Q4 block
    (129, 64, 160, None),
    # K % 64 == 0 takes the DMA-pipelined kernel: ragged tokens and features,
    # and fewer K steps (1, 2, 3) than DMA groups in flight
    (100, 200, 128, None),
    (1, 70, 64, None),
    (257, 100, 192, None),
    (130, 64, 448, None),
])
def test_batch_gemm_q4_parity(ctx, n_tok, M, K, sample):
    seed = 9000 + n_tok + M + K
    W = synth_q4_dev(ctx, M, K, seed)
    X = synth_normal_dev(ctx, n_tok * K, seed + 1)
    Y = ctx.alloc(n_tok * M * 4)
    say(f"batch_gemm_q4 n_tok={n_tok} M={M} K={K}")
    ctx.call("chn_batch_gemm_q4", W, X, Y, n_tok, M, K)
    Yg = f32_host(ctx, Y, n_tok * M).reshape(n_tok, M)
    Xh = f32_host(ctx, X, n_tok * K).reshape(n_tok, K)
    Wh = q4_host(ctx, W, M, K)
    rows = np.arange(n_tok) if sample is None else np.unique(
        np.concatenate([[0, n_tok - 1], np.random.default_rng(seed).integers(0, n_tok, sample)]))
    Xs = np.ascontiguousarray(Xh[rows])
    want16 = oracle.batch_gemm_q4_bf16(Wh, Xs, len(rows), M, K)
    want32 = oracle.batch_gemm_q4(Wh, Xs, len(rows), M, K)
    assert rel_err(Yg[rows], want16) < 1e-4
    assert rel_err(Yg[rows], want32) < 1e-2


@pytest.mark.parametrize("n_tok,M,K,sample", [
    (512, 15360, 3840, 8),     # batched fused MLP at 12B dims
    (70, 96, 128, None),
])
def test_batch_fused_mlp_q4_parity(ctx, n_tok, M, K, sample):
    seed = 9500 + n_tok + M
    Wg = synth_q4_dev(ctx, M, K, seed)
    Wu = synth_q4_dev(ctx, M, K, seed + 1)
    X = synth_normal_dev(ctx, n_tok * K, seed + 2)
    Y = ctx.alloc(n_tok * M * 4)
    say(f"batch_fused_mlp_q4 n_tok={n_tok} M={M} K={K}")
    ctx.call("chn_batch_fused_mlp_q4", Wg, Wu, X, Y, n_tok, M, K)
    Yg = f32_host(ctx, Y, n_tok * M).reshape(n_tok, M)
    Xh = f32_host(ctx, X, n_tok * K).reshape(n_tok, K)
    rows = np.arange(n_tok) if sample is None else np.unique(
        np.concatenate([[0, n_tok - 1], np.random.default_rng(seed).integers(0, n_tok, sample)]))
    Xs = np.ascontiguousarray(Xh[rows])
    Wgh, Wuh = q4_host(ctx, Wg, M, K), q4_host(ctx, Wu, M, K)
    want = oracle.batch_fused_mlp_q4(Wgh, Wuh, Xs, len(rows), M, K)
    assert rel_err(Yg[rows], want) < 1e-2
    g16 = oracle.batch_gemm_q4_bf16(Wgh, Xs, len(rows), M, K)
    u16 = oracle.batch_gemm_q4_bf16(Wuh, Xs, len(rows), M, K)
    want16 = np.array([oracle.gelu_tanh(r) for r in g16]) * u16
    assert rel_err(Yg[rows], want16) < 1e-4
