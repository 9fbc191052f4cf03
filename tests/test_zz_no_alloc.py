"""The allocation-free GEMM (vdn_fp8_gemm_noalloc) against the GEMM with a caller-provided
workspace (vdn_fp8_gemm_ws) through the C ABI: the same kernels with the split-K partial
sums in the library's static device array instead of the caller's buffer, so every output
must be bit-identical. Two calls in a row, the second with a smaller input (its split reads
only what it wrote itself), then a shape that does not split."""
import pytest
import torch

import vdn_fp8
import vdn_fp8._lib as L

pytestmark = pytest.mark.gpu


def _setup(device, M, N, K, seed, bias=True):
    g = torch.Generator().manual_seed(seed)
    qx, sx = vdn_fp8.quantize_rows(torch.randn(M, K, generator=g).to(torch.bfloat16).to(device))
    lin = torch.nn.Linear(K, N, bias=bias, dtype=torch.bfloat16, device="meta")
    lin.weight = torch.nn.Parameter((0.02 * torch.randn(N, K, generator=g)).to(torch.bfloat16).to(device),
                                    requires_grad=False)
    lin.bias = torch.nn.Parameter((0.01 * torch.randn(N, generator=g)).to(torch.bfloat16).to(device),
                                  requires_grad=False) if bias else None
    return vdn_fp8.Fp8Linear(lin), qx, sx


def _call(entry, f, qx, sx, epi=0, gate=None, gi=None, grows=0, res=None, ws=None):
    lib = L.load()
    M, K = qx.shape
    N = f.weight_fp8.shape[0]
    out = torch.empty(M, N, dtype=torch.bfloat16, device=qx.device)
    ptr = lambda t: None if t is None else t.data_ptr()
    b = f.bias.detach() if f.bias is not None else None
    args = (ptr(qx), ptr(sx), ptr(f.weight_fp8), ptr(f.weight_scale), M, N, K, K, K, ptr(b), epi, ptr(gate), ptr(gi),
            grows, 0 if gate is None else gate.stride(0), ptr(res), 0 if res is None else res.stride(0), ptr(out), N)
    st = torch.cuda.current_stream(qx.device).cuda_stream
    if entry == "ws":
        L.check(lib.vdn_fp8_gemm_ws(*args, ptr(ws), 0 if ws is None else ws.numel(), st), "gemm_ws")
    else:
        L.check(lib.vdn_fp8_gemm_noalloc(*args, st), "gemm_noalloc")
    return out


def _ws(device, M, N, K):
    n = vdn_fp8.fp8_linear.gemm_workspace_bytes(M, N, K, device)
    return torch.empty(n, dtype=torch.uint8, device=device) if n else None


def test_noalloc_matches_the_workspace_entry_point(device):
    # call 1: the H3 FF down projection, 13107 x 5376 x 14336 (68 tiles of the last round
    # split three ways: 51 MiB of partial sums), gate table by row and a residual
    M, N, K = 13107, 5376, 14336
    print(f"noalloc call 1: {M} x {N} x {K}, gate rows + residual", flush=True)
    f, qx, sx = _setup(device, M, N, K, 1, bias=False)
    g = torch.Generator().manual_seed(2)
    gate = (2 * torch.rand(4, N, generator=g)).to(torch.bfloat16).to(device)
    gi = torch.randint(0, 4, (M,), generator=g).to(torch.int32).to(device)
    res = torch.randn(M, N, generator=g).to(torch.bfloat16).to(device)
    assert vdn_fp8.fp8_linear.gemm_workspace_bytes(M, N, K, device) > 0
    kw = dict(epi=L.EPI_GATE, gate=gate, gi=gi, grows=4, res=res)
    want = _call("ws", f, qx, sx, ws=_ws(device, M, N, K), **kw)
    got = _call("noalloc", f, qx, sx, **kw)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    # call 2, smaller: 700 x 1024 x 8192 with bias and GELU (12 tiles, eight slices each)
    M, N, K = 700, 1024, 8192
    print(f"noalloc call 2: {M} x {N} x {K}, bias + gelu", flush=True)
    f, qx, sx = _setup(device, M, N, K, 3)
    assert vdn_fp8.fp8_linear.gemm_workspace_bytes(M, N, K, device) > 0
    want = _call("ws", f, qx, sx, epi=L.EPI_GELU_TANH, ws=_ws(device, M, N, K))
    got = _call("noalloc", f, qx, sx, epi=L.EPI_GELU_TANH)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    # a shape that does not split: the same as the plain entry point
    M, N, K = 1000, 768, 5120
    print(f"noalloc call 3: {M} x {N} x {K}, no split", flush=True)
    f, qx, sx = _setup(device, M, N, K, 4)
    assert vdn_fp8.fp8_linear.gemm_workspace_bytes(M, N, K, device) == 0
    want = _call("ws", f, qx, sx)
    got = _call("noalloc", f, qx, sx)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
