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
  dit_lora    base W [15360, 5120] + rank-64 LoRA (alpha 64) and the block input X, seed 5
  dit_block   one block's four linears: the LoRA-merged QKV on dit_lora's X, attention-out,
              FFN-up + GELU and FFN-down + gate with the other draws' weights
M = 32760 is 21 latent frames x 30 x 52 patches. DRAW_SHA256 pins every full-size draw.
"""
import hashlib
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


def dit_block(M=TOKENS):
    """One DiT block's four fp8 linears as the LoRA workload runs them (seed 5 for the
    block input): the QKV weight is dit_lora's base weight with its rank-64 LoRA folded in
    and dit_qkv's bias; attention-out and FFN-down are dit_ffn_down_attn_out's weights
    with its AdaLN gate; FFN-up is dit_ffn_up's weight and bias with GELU(tanh). The
    weights are those of the full-size draws (each draw sequence puts X first).

    Returns a dict: x, w0, a, b, lora_scale, qkv_bias, w_out, w_up, b_up, w_down, gate."""
    w0, a, b, scale, x = dit_lora(M)
    _, _, qkv_bias = dit_qkv()
    _, w_up, b_up = dit_ffn_up()
    (_, w_down), (_, w_out), gate = dit_ffn_down_attn_out()
    return dict(x=x, w0=w0, a=a, b=b, lora_scale=scale, qkv_bias=qkv_bias, w_out=w_out, w_up=w_up,
                b_up=b_up, w_down=w_down, gate=gate)


def sha256(t):
    """sha256 of a bf16 tensor's bytes (row-major)."""
    return hashlib.sha256(t.contiguous().view(torch.int16).numpy().tobytes()).hexdigest()


# sha256 of every full-size draw, as produced by torch's CPU generator: a change in that
# generator would silently change the inputs, so the tests (and bench.py, for the draw
# it times) compare against these.
DRAW_SHA256 = {
    "dit_single": {"x": "8e8dc87032770e08a7228dff86a712858bdcd5089cecfb901288a8fe13f0fdd9",
                   "w": "515a2c50911ca96b8883b89377e7db69cac7423a78022cb4c58fa6e69d58bada",
                   "bias": "532e5ad6a60179f156d6229a1c6a0e70649edc728f4ce7722babf51667d3324d"},
    "dit_qkv": {"x": "0c0a840a1ab0af5cb382df53c6e28b1657190f77d990e995d0602474093d2678",
                "w": "0f49aa9c88fa2b7956c3e81865ead449000b5c35e7fbd0d5c99b16fa320c9387",
                "bias": "5360751a55d281f20d5069870a5cb5ed67b14c331d0ccf7572915dd071abd56c"},
    "dit_ffn_up": {"x": "7b9febb793e8d1151ed607cffaa2a1e7e7e7d28fc5b8d35d178de56654c73ea9",
                   "w": "a8ecdee89261d83ba0a92756dfb97549d3e9a8a872f0abc7ab831aea6eef7a13",
                   "bias": "551f311f154c91fe07f6d46a2266927904b30c0d35d4922ed0b314845cf67dd6"},
    "dit_ffn_down_attn_out": {
        "x_down": "f195bfe7277b163a66cc6ee0863b24d7444a9db4adfdb5868f845525a6acc926",
        "w_down": "7be0305d6f91aa57122eb120a50c52e6f0fe406e00b1d478a395ce52e1826e03",
        "x_out": "3e374368b6397ebb54e920bbfe5e3ca6c14c99faf439d358ba0dd797583fc4a4",
        "w_out": "3a8536abe77a0c17ffd190fc06d4e92289f6ded5e29520c1e6daef52ff0838a1",
        "gate": "1ab8c931a0631faa1d3ff13e2da05b99122abd459b6c6525ba02c0ee9873e9f6"},
    "dit_lora": {"w0": "bd0f8d8337f9862fdcd4874ea6dae77d0149757bd7afb2df07c450089333c7ab",
                 "a": "3d3702eb604642b0b0114c2dac4f44d432286d9fb3b01ccc9c64d18770ed4ca4",
                 "b": "ba3d42d6bdad5de59590e92647618d05e64ed5138fec8fea7993cc9e9945fb80",
                 "x": "526126abe828819e58d110725fa2db6708898792d63443da42ff416abc56d494"},
}


def draw_digests(name):
    """{tensor: sha256} of the full-size draw `name` (a key of DRAW_SHA256)."""
    if name == "dit_ffn_down_attn_out":
        (xd, wd), (xo, wo), g = dit_ffn_down_attn_out()
        named = dict(x_down=xd, w_down=wd, x_out=xo, w_out=wo, gate=g)
    elif name == "dit_lora":
        w0, a, b, _, x = dit_lora()
        named = dict(w0=w0, a=a, b=b, x=x)
    else:
        x, w, b = globals()[name]()
        named = dict(x=x, w=w, bias=b)
    return {k: sha256(v) for k, v in named.items()}
