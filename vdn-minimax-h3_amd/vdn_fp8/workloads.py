"""Seeded synthetic inputs of the DiT fp8-linear shapes that the benchmark and the
parity tests run (no datasets or checkpoints are involved).

Every tensor is drawn on the CPU with torch.Generator(seed), in fp32 and in the order
listed, scaled, then rounded to bf16 -- so the same seed gives the same bits on any
machine whose torch CPU generator matches (tests pin the sha256 of the draws).

  dit_single  [1024 x 1024 x 1024] one linear, seed 0
  dit_qkv     X [32760, 5120] ~N(0,1) with 5 outlier channels x20, fused QKV W [15360, 5120]
  dit_ffn_up  X [32760, 5120], W [13824, 5120], bias, GELU(tanh)
  dit_ffn_down / dit_attn_out   X [32760, 13824] = gelu(N(0,1)) / X [32760, 5120], W [5120, *],
                                AdaLN gate [5120] ~ 2 U(0,1)
  dit_lora    base W [15360, 5120] + rank-64 LoRA (alpha 64), then a block's four linears
M = 32760 is 21 latent frames x 30 x 52 patches.
"""
import math

import torch

TOKENS = 32760
HIDDEN = 5120
QKV = 3 * HIDDEN
FFN = 13824
LORA_RANK = 64
LORA_ALPHA = 64.0


def _gen(seed):
    return torch.Generator("cpu").manual_seed(seed)


def _normal(g, shape, std=1.0):
    return torch.randn(*shape, generator=g, dtype=torch.float32) * std


def gelu_tanh_f32(x):
    c = math.sqrt(2.0 / math.pi)
    return 0.5 * x * (1.0 + torch.tanh(c * (x + 0.044715 * x * x * x)))


def linear_inputs(seed, M, N, K, outliers=0, bias=True, x_gelu=False):
    """X bf16 [M, K], W bf16 [N, K] ~ 0.02 N(0,1), bias bf16 [N] ~ 0.01 N(0,1) (or None).

    Draw order: X, (outlier channel permutation), W, bias."""
    g = _gen(seed)
    x = _normal(g, (M, K))
    if x_gelu:
        x = gelu_tanh_f32(x)
    if outliers:
        ch = torch.randperm(K, generator=g)[:outliers]
        x[:, ch] *= 20.0
    x = x.to(torch.bfloat16)
    w = _normal(g, (N, K), 0.02).to(torch.bfloat16)
    b = _normal(g, (N,), 0.01).to(torch.bfloat16) if bias else None
    return x, w, b


def dit_single():
    """Single fp8 linear [1024 x 1024 x 1024], seed 0."""
    return linear_inputs(0, 1024, 1024, 1024)


def dit_qkv(M=TOKENS):
    """Fused QKV projection: 0.1% of the 5120 channels (5) scaled x20, seed 2."""
    return linear_inputs(2, M, QKV, HIDDEN, outliers=5)


def dit_ffn_up(M=TOKENS):
    """FFN up-projection with bias, GELU(tanh) epilogue, seed 3."""
    return linear_inputs(3, M, FFN, HIDDEN)


def dit_ffn_down_attn_out(M=TOKENS):
    """FFN down (X = gelu(N(0,1))) and attention-out projections, AdaLN gate, seed 4.

    Returns (x_down, w_down), (x_out, w_out), gate [5120]. No bias, no residual."""
    g = _gen(4)
    x_down = gelu_tanh_f32(_normal(g, (M, FFN))).to(torch.bfloat16)
    w_down = _normal(g, (HIDDEN, FFN), 0.02).to(torch.bfloat16)
    x_out = _normal(g, (M, HIDDEN)).to(torch.bfloat16)
    w_out = _normal(g, (HIDDEN, HIDDEN), 0.02).to(torch.bfloat16)
    gate = (2.0 * torch.rand(HIDDEN, generator=g, dtype=torch.float32)).to(torch.bfloat16)
    return (x_down, w_down), (x_out, w_out), gate


def dit_lora(M=TOKENS):
    """Base QKV weight + rank-64 LoRA (alpha 64 -> scale 1.0) and the block input, seed 5.

    Returns w0 [15360, 5120], a [64, 5120], b [15360, 64], scale, x [M, 5120]."""
    g = _gen(5)
    w0 = _normal(g, (QKV, HIDDEN), 0.02).to(torch.bfloat16)
    a = _normal(g, (LORA_RANK, HIDDEN), 0.01).to(torch.bfloat16)
    b = _normal(g, (QKV, LORA_RANK), 0.01).to(torch.bfloat16)
    x = _normal(g, (M, HIDDEN)).to(torch.bfloat16)
    return w0, a, b, LORA_ALPHA / LORA_RANK, x


def linear_flops(M, N, K):
    return 2.0 * M * N * K


def quant_bytes(M, K):
    """Algorithmic HBM bytes of a row quantization: bf16 in, e4m3 out, fp32 scale per row."""
    return 2.0 * M * K + M * K + 4.0 * M


def requant_bytes(N, K, rank=0):
    """Algorithmic HBM bytes of a weight requantization (+ LoRA factors when fused)."""
    return 2.0 * N * K + N * K + 4.0 * N + (2.0 * rank * (N + K) if rank else 0.0)
