"""Benchmark of the fp8 quantized-linear path on one MI355X.

    python bench.py [--gpus 1] [--steps 20] [--warmup 50] [--no-cpu-baseline] [--no-extra]
    python bench.py --only NAME [--steps K] [--warmup W]     # one kernel's workload, for profilers

A step is one pass of the hot path over the DiT QKV projection: per-token e4m3
quantization of X [32760, 5120] followed by the fp8 GEMM against the fused QKV weight
[15360, 5120] with per-token x per-channel dequantization and the bias fused in. Inputs
are synthetic (seeded, their sha256 checked), resident in HBM before the timed region.
Prints ONE JSON line:

  value       whole-step throughput, 2*M*N*K / step time (TFLOP/s)
  roofline    the GEMM kernel alone, from HIP events on the stream it runs on, against
              the dense fp8 MFMA peak (5.03 PFLOP/s); `traffic` (HBM bytes per launch) and
              the MFMA-busy / clock counters come from the committed rocprofv3 profile of
              this same kernel, and are null when that profile was taken of other code
  cpu_baseline  the oracle on this host's cores: the single linear (median of 3), and
              every config's kernel-equivalents at full size
  extra       the quantizer's HBM rate, the weight requantizer (plain and with the fused
              rank-64 LoRA merge), the other DiT GEMMs, the ms of one block's four
              linears, the H3-width shapes and the pointwise kernels; each HBM-bound
              kernel also against a bare read + write stream of its own bytes
              (`stream_GB/s`, `of_stream`), the rate this part gives for that traffic
"""
import argparse
import functools
import itertools
import json
import os
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "vdn-minimax-h3_amd"))

METRIC = "fp8 linear TFLOP/s & % fp8 MFMA peak (M=32760 QKV); ms per DiT-block linears"
PEAK_FP8_TFLOPS = 5030.0     # 256 CU x 2.4 GHz x 8192 FLOP/clk/CU, dense
NOMINAL_GHZ = 2.4
PEAK_HBM_GBPS = 8000.0
PROFILE = os.path.join(ROOT, "profiles", "gemm_qkv_pmc.json")


def _events(n):
    import torch
    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


def _gpu_clock():
    try:
        r = subprocess.run(["rocm-smi", "--showclocks"], capture_output=True, text=True, timeout=20)
        lines = [l.strip() for l in r.stdout.splitlines() if "sclk" in l.lower()]
        return lines[0] if lines else None
    except Exception:
        return None


def _smi_sample():
    """(mean graphics clock over the XCDs in MHz, socket power in W) from amd-smi, or None."""
    try:
        r = subprocess.run(["amd-smi", "metric", "-c", "-p", "--json"], capture_output=True, text=True, timeout=10)
        d = json.loads(r.stdout)
        g = d["gpu_data"][0] if isinstance(d, dict) else d[0]
        clks = [v["clk"]["value"] for k, v in g.get("clock", {}).items()
                if k.startswith("gfx_") and isinstance(v, dict) and isinstance(v.get("clk"), dict)]
        pw = g.get("power", {}).get("socket_power", {})
        return (sum(clks) / len(clks) if clks else None, pw.get("value") if isinstance(pw, dict) else None)
    except Exception:
        return None


def _under_load(fn, seconds=2.0):
    """Runs fn back to back for about `seconds` while a thread samples amd-smi: the clock the
    part sustains on this work and the power it draws (the clock falls when the power limit
    binds)."""
    import threading
    import torch
    samples, stop = [], threading.Event()

    def sampler():
        time.sleep(0.3)                      # let the clock settle under the load
        while not stop.is_set():
            smp = _smi_sample()
            if smp is None:
                return
            samples.append(smp)

    th = threading.Thread(target=sampler, daemon=True)
    t_end = time.perf_counter() + seconds
    th.start()
    while time.perf_counter() < t_end:
        for _ in range(25):
            fn()
        torch.cuda.synchronize()
    stop.set()
    th.join(timeout=15)
    clk = [c for c, _ in samples if c]
    pw = [w for _, w in samples if w]
    if not clk:
        return None
    return {"gfx_mhz": round(sum(clk) / len(clk)), "gfx_mhz_min": round(min(clk)),
            "socket_w": round(sum(pw) / len(pw)) if pw else None, "samples": len(clk)}


WARM_MS = 60.0


def _warm(*fns, ms=WARM_MS):
    """Runs the given calls for at least `ms` of wall time before a timed region: the
    part lowers its clock while the host prepares inputs, and needs some tens of
    milliseconds of load to raise it again (a 1.2 ms GEMM timed right after such a
    pause reads ~15% slow over its first dozen launches)."""
    import torch
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(4):
            for f in fns:
                f()
        torch.cuda.synchronize()


def _time_pair(fa, fb, reps):
    """Mean ms of fa() and of fb(), launched alternately (a, b, a, b, ...) so that a clock
    that drifts while the part heats up weighs on both alike (after a warm-up)."""
    import torch
    _warm(fa, fb)
    ev = _events(4 * reps)
    for i in range(reps):
        ev[4 * i].record()
        fa()
        ev[4 * i + 1].record()
        fb()
        ev[4 * i + 2].record()
    torch.cuda.synchronize()
    ta = sum(ev[4 * i].elapsed_time(ev[4 * i + 1]) for i in range(reps)) / reps
    tb = sum(ev[4 * i + 1].elapsed_time(ev[4 * i + 2]) for i in range(reps)) / reps
    return ta, tb


def _time_region(fn, reps):
    """Mean ms of fn() over reps launches, from HIP events on the current stream (after a
    warm-up of untimed calls)."""
    import torch
    _warm(fn)
    ev = _events(2 * reps)
    for i in range(reps):
        ev[2 * i].record()
        fn()
        ev[2 * i + 1].record()
    torch.cuda.synchronize()
    return sum(ev[2 * i].elapsed_time(ev[2 * i + 1]) for i in range(reps)) / reps


def _probe_lib():
    """The measurement probes (bare stream, bare MFMA loop; built beside libvdnfp8.so), or
    None if absent."""
    import ctypes
    path = os.path.join(ROOT, "vdn-minimax-h3_amd", "vdn_fp8", "libvdnprobe.so")
    if not os.path.exists(path):
        return None
    lib = ctypes.CDLL(path)
    P, I = ctypes.c_void_p, ctypes.c_int
    lib.vdn_stream_probe.argtypes = [I, I, I, P, ctypes.c_int64, P, I, P]
    lib.vdn_stream_probe.restype = I
    lib.vdn_mfma_probe.argtypes = [I, P, P, ctypes.c_int64, ctypes.c_int64, I, I, P, P]
    lib.vdn_mfma_probe.restype = I
    return lib


def _mfma_ceiling(lib, xq, wq, blocks, grid, reps):
    """The bare fp8 MFMA loop (the GEMM's grid, instruction and LDS fragment reads, no
    copies, no epilogue) on the GEMM's own codes, on uniform codes, and with the fragments
    held in registers, and the 32 x 32 x 64 instruction on the same codes: ms, TFLOP/s,
    fraction of the dense peak, and the clock and power amd-smi reads while it runs back to
    back."""
    import ctypes
    import torch
    out = torch.empty(grid * 256, dtype=torch.float32, device=xq.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    flop = grid * 4 * blocks * 32 * (2 * 32 * 32 * 64)
    tiles = min(xq.shape[0], wq.shape[0]) // 256
    res = {"instruction": "v_mfma_f32_16x16x128_f8f6f4 (the GEMM's)"}
    for name, mode in (("random_codes", 3), ("uniform_codes", 4), ("random_codes_registers_only", 5),
                       ("v_mfma_f32_32x32x64_f8f6f4_random_codes", 0)):
        def call():
            rc = lib.vdn_mfma_probe(mode, ctypes.c_void_p(xq.data_ptr()), ctypes.c_void_p(wq.data_ptr()),
                                    xq.stride(0), tiles, blocks, grid, ctypes.c_void_p(out.data_ptr()), stream)
            if rc:
                raise RuntimeError(f"vdn_mfma_probe failed ({rc})")
        ms = _time_region(call, reps)
        tf = flop / (ms * 1e-3) / 1e12
        res[name] = {"ms": round(ms, 4), "TFLOP/s": round(tf, 1), "frac": round(tf / PEAK_FP8_TFLOPS, 4),
                     "under_load": _under_load(call, seconds=1.5)}
    res["flop"] = flop
    return res


def _torch_rate(read_bytes, write_bytes, rotate=1, reps=10):
    """GB/s of a torch library kernel moving a kernel's bytes with the same read : write
    ratio: copy_ (1:1), torch.add(a, b, out=c) (2:1), torch.sum over groups of four (4:1),
    on bf16 tensors, the sources rotated over `rotate` disjoint copies when the kernel's
    input is (so that it comes from HBM)."""
    import torch
    kr = max(1, round(read_bytes / write_bytes))
    n = int(write_bytes // 2) // 256 * 256          # bf16 elements written
    dev = torch.device("cuda:0")
    dst = torch.empty(n, dtype=torch.bfloat16, device=dev)
    srcs = [torch.empty(kr * n, dtype=torch.bfloat16, device=dev).normal_() for _ in range(rotate)]
    rot = itertools.cycle(srcs)
    if kr == 1:
        fn = lambda: dst.copy_(next(rot))
    elif kr == 2:
        def fn():
            s_ = next(rot)
            torch.add(s_[:n], s_[n:], out=dst)
    elif kr == 4:
        fn = lambda: torch.sum(next(rot).view(-1, 4, 256), dim=1, out=dst.view(-1, 256))
    else:
        raise ValueError(f"no torch kernel for a {kr}:1 mix")
    ms = _time_region(fn, reps)
    del srcs, dst
    return (kr * n * 2 + n * 2) / (ms * 1e-3) / 1e9


def _stream_rate(lib, src, dst, read_bytes, write_bytes, nt_store, rotate=1, reps=10):
    """GB/s of a bare stream moving a kernel's bytes: read_bytes read and write_bytes
    written (1 KiB pieces, the read : write ratio rounded to 1, 2 or 4), stores
    non-temporal or cached as the kernel's are, the source rotated over `rotate` disjoint
    copies when the kernel's input is (so that it comes from HBM). Best of four grid
    sizes, each timed as the kernels are (_time_region)."""
    import ctypes
    import torch
    kr = max(1, round(read_bytes / write_bytes))
    units = int(write_bytes // 1024)
    rb, wb = units * kr * 1024, units * 1024
    if rotate * rb > src.numel() or wb > dst.numel():
        raise ValueError("stream probe buffers too small")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    best = 0.0
    for grid in (1024, 2048, 4096, 8192):
        srcs = itertools.cycle([src.data_ptr() + i * rb for i in range(rotate)])

        def call():
            rc = lib.vdn_stream_probe(kr, 1, int(nt_store), ctypes.c_void_p(next(srcs)), units,
                                      ctypes.c_void_p(dst.data_ptr()), grid, stream)
            if rc:
                raise RuntimeError(f"vdn_stream_probe failed ({rc})")
        ms = _time_region(call, reps)
        best = max(best, (rb + wb) / (ms * 1e-3) / 1e9)
    return best


def _make_linear(w, b, dev, lora=None):
    import torch
    import vdn_fp8
    lin = torch.nn.Linear(w.shape[1], w.shape[0], bias=b is not None, dtype=torch.bfloat16, device="meta")
    lin.weight = torch.nn.Parameter(w.to(dev), requires_grad=False)
    lin.bias = torch.nn.Parameter(b.to(dev), requires_grad=False) if b is not None else None
    return vdn_fp8.Fp8Linear(lin, lora=lora)


# ---------------------------------------------------------------------------------------
# CPU baseline: the oracle (the reference's eager CPU spelling, restated) on host cores
# ---------------------------------------------------------------------------------------

def cpu_baseline(draws):
    """The reference's CPU path, restated by the oracle, timed on this host: C row and
    weight quantizers and LoRA merge (pthreads), numpy binary32 dequantized matmul plus
    the epilogue (BLAS threads). cfg1 (the single 1024^3 linear): quantize X, quantize W,
    matmul + bias, median of 3 after one warm-up. cfg2-5: each kernel-equivalent once at
    full size. `value` is the QKV step (quantize X + matmul + bias) in TFLOP/s."""
    import numpy as np
    import torch
    from threadpoolctl import threadpool_limits

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    from vdn_fp8 import workloads as wl
    cores = min(16, os.cpu_count() or 1)
    os.environ["ORACLE_THREADS"] = str(cores)

    def u16(t):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)

    def deq(q, s):
        return O.e4m3_decode(q) * s[:, None]

    def gelu(v):
        return 0.5 * v * (1.0 + np.tanh(np.float32(0.7978845608028654) * (v + np.float32(0.044715) * v * v * v)))

    def timed(fn):
        t0 = time.perf_counter()
        r = fn()
        return r, (time.perf_counter() - t0) * 1e3

    per = {}
    with threadpool_limits(limits=cores):
        x, w, b = (u16(t) for t in wl.dit_single())

        def single():
            qx, sx = O.quantize_rows(x)
            qw, sw = O.quantize_weight(w)
            return deq(qx, sx) @ deq(qw, sw).T + O.bf16_decode(b)[None, :]
        single()
        runs = [timed(single)[1] for _ in range(3)]
        per["cfg1_single_linear_ms"] = round(statistics.median(runs), 3)

        def linear(name, xb, wb, bias=None, epi=None, gate=None):
            (qx, sx), tq = timed(lambda: O.quantize_rows(xb))
            (qw, sw), tw = timed(lambda: O.quantize_weight(wb))
            def mm():
                out = deq(qx, sx) @ deq(qw, sw).T
                if bias is not None:
                    out += O.bf16_decode(bias)[None, :]
                if epi == "gelu_tanh":
                    out = gelu(out)
                elif epi == "gate":
                    out *= O.bf16_decode(gate)[None, :]
                return out
            _, tg = timed(mm)
            per[name] = {"quantize_x_ms": round(tq, 1), "quantize_w_ms": round(tw, 1), "gemm_epilogue_ms": round(tg, 1)}
            return tq, tg

        tq, tg = linear("cfg2_qkv", draws["x2"], draws["w2"], draws["b2"])
        value = wl.linear_flops(*draws["x2"].shape[:1], draws["w2"].shape[0], draws["x2"].shape[1]) / ((tq + tg) * 1e-3) / 1e12
        linear("cfg3_ffn_up_gelu", draws["x3"], draws["w3"], draws["b3"], "gelu_tanh")
        linear("cfg4_ffn_down_gate", draws["x4d"], draws["w4d"], None, "gate", draws["g4"])
        linear("cfg4_attn_out_gate", draws["x4o"], draws["w4o"], None, "gate", draws["g4"])
        wm, tm = timed(lambda: O.lora_merge(draws["w5"], draws["a5"], draws["b5"], draws["s5"]))
        _, tw = timed(lambda: O.quantize_weight(wm))
        per["cfg5_lora_merge_requantize"] = {"merge_ms": round(tm, 1), "quantize_w_ms": round(tw, 1)}
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = None
    return {"value": round(value, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "host_cpu_count": os.cpu_count(), "affinity_cpus": affinity,
            "threads_note": "threads = min(16, os.cpu_count()): the host's CPU share is 16 per GPU",
            "sample": "the whole QKV step (quantize X [32760, 5120], dequantized fp32 matmul against W "
                      "[15360, 5120] + bias) once at full size; cfg1 median of 3 after a warm-up; the other "
                      "configs' kernel-equivalents once each at full size (oracle C quantizers and merge, numpy "
                      "fp32 matmul)",
            "per_config": per}


# ---------------------------------------------------------------------------------------
# the committed profile of the GEMM, used only when it was taken of the code loaded now
# ---------------------------------------------------------------------------------------

def _profile_fields():
    """(traffic, counters) from profiles/gemm_qkv_pmc.json when its kernel digest equals the
    loaded library's GEMM digest, else (None, {"stale": ...})."""
    import vdn_fp8._lib as L
    from vdn_fp8 import build as B
    digest = B.kernel_digest(L.build_info(), "gemm")
    if not os.path.exists(PROFILE):
        return None, {"profile": None}
    with open(PROFILE) as f:
        prof = json.load(f)
    if prof.get("kernel_digest") != digest:
        return None, {"profile": os.path.relpath(PROFILE, ROOT),
                      "stale": "profiled code differs from the loaded GEMM (digest mismatch)"}
    c = prof["counters"]
    return prof["traffic_bytes"], {
        "profile": os.path.relpath(PROFILE, ROOT), "kernel_digest": digest[:16],
        "mfma_busy_per_active_cycle": c["mfma_busy_per_active_cycle"],
        "effective_clock_ghz": c["effective_clock_ghz"],
        "frac_at_effective_clock": c["frac_at_effective_clock"]}


# ---------------------------------------------------------------------------------------
# single-workload mode (one kernel's launches, for rocprofv3 runs)
# ---------------------------------------------------------------------------------------

def _only(name, steps, warmup):
    import torch
    import vdn_fp8
    from vdn_fp8 import fused_block as FB
    from vdn_fp8 import workloads as wl
    dev = torch.device("cuda:0")
    if name in ("lora_requant", "requant"):
        w0, a, b, scale, _ = wl.dit_lora(M=8)
        copies = [w0.to(dev) for _ in range(3)]
        rot = itertools.cycle(copies)
        lora = (a.to(dev), b.to(dev), scale) if name == "lora_requant" else None
        fn = lambda: vdn_fp8.requantize_weight(next(rot), lora=lora)
    elif name in ("quantize_13824", "quantize_5120"):
        x = torch.empty(wl.TOKENS, int(name.split("_")[1]), dtype=torch.bfloat16, device=dev).normal_()
        fn = lambda: vdn_fp8.quantize_rows(x)
    elif name == "swiglu_h3":
        h = torch.empty(wl.TOKENS, 2 * 14336, dtype=torch.bfloat16, device=dev).normal_()
        fn = lambda: vdn_fp8.swiglu_quantize(h)
    elif name in ("pre_norm_quantize", "pre_norm_quantize_h3"):
        M_, K_, T_ = (wl.TOKENS, wl.HIDDEN, 21) if name == "pre_norm_quantize" else (13107, 5376, 5)
        x = torch.empty(M_, K_, dtype=torch.bfloat16, device=dev).normal_()
        nw = torch.ones(K_, dtype=torch.bfloat16, device=dev)
        tab = (0.2 * torch.randn(T_, K_, device=dev)).to(torch.bfloat16)
        idx = (torch.arange(M_, device=dev) * T_ // M_).to(torch.int32)
        fn = lambda: FB.pre_quantize(x, nw, 1e-6, tab, tab, idx)
    elif name == "post":
        x = torch.empty(wl.TOKENS, wl.HIDDEN, dtype=torch.bfloat16, device=dev).normal_()
        br = torch.empty_like(x).normal_()
        gt = (2 * torch.rand(2, wl.HIDDEN, device=dev)).to(torch.bfloat16)
        gid = torch.randint(0, 2, (wl.TOKENS,), device=dev)
        fn = lambda: FB.post(x, gt, gid, br)
    elif name == "qk_prep":
        y = torch.empty(wl.TOKENS, 3 * wl.HIDDEN, dtype=torch.bfloat16, device=dev).normal_()
        qv = y[:, :wl.HIDDEN].unflatten(-1, (40, 128))
        nq = torch.ones(128, dtype=torch.bfloat16, device=dev)
        th = torch.rand(wl.TOKENS, 64, device=dev) * 6.28
        cs, sn = torch.cat([th.cos(), th.cos()], 1), torch.cat([th.sin(), th.sin()], 1)
        fn = lambda: vdn_fp8.qk_prep(qv, nq, 1e-6, cs, sn)
    elif name in ("gemm_h3_ff_down", "gemm_qkv"):
        M_, N_, K_ = (13107, 5376, 14336) if name == "gemm_h3_ff_down" else (wl.TOKENS, wl.QKV, wl.HIDDEN)
        gh = torch.Generator().manual_seed(13)
        qx, sx = vdn_fp8.quantize_rows(torch.randn(M_, K_, generator=gh).to(torch.bfloat16).to(dev))
        lin = _make_linear((0.02 * torch.randn(N_, K_, generator=gh)).to(torch.bfloat16), None, dev)
        fn = lambda: lin.forward_quantized(qx, sx)
    else:
        raise SystemExit(f"unknown --only workload {name!r}")
    for _ in range(warmup):
        fn()
    ms = _time_region(fn, steps)
    print(json.dumps({"only": name, "steps": steps, "warmup": warmup, "ms": round(ms, 4)}), flush=True)


# ---------------------------------------------------------------------------------------

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--only", default=None, help="time one workload's kernel alone (lora_requant, requant, "
                    "quantize_5120, quantize_13824, swiglu_h3, pre_norm_quantize, pre_norm_quantize_h3, post, qk_prep, "
                    "gemm_h3_ff_down, "
                    "gemm_qkv)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the fp8 linear path has no cross-GPU step "
              f"(rows shard without exchange); --gpus {args.gpus} is not run.", file=sys.stderr)
        sys.exit(2)
    if args.only:
        return _only(args.only, args.steps, args.warmup)

    import torch
    import vdn_fp8
    from vdn_fp8 import workloads as wl

    dev = torch.device("cuda:0")
    x_cpu, w_cpu, b_cpu = wl.dit_qkv()
    inputs_ok = {"x": wl.sha256(x_cpu), "w": wl.sha256(w_cpu), "bias": wl.sha256(b_cpu)} == wl.DRAW_SHA256["dit_qkv"]
    M, K = x_cpu.shape
    N = w_cpu.shape[0]
    x = x_cpu.to(dev)
    lin = _make_linear(w_cpu, b_cpu, dev)

    def step():
        qx, sx = vdn_fp8.quantize_rows(x)
        return lin.forward_quantized(qx, sx)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    ev = _events(3 * args.steps)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        ev[3 * i].record()
        qx, sx = vdn_fp8.quantize_rows(x)
        ev[3 * i + 1].record()
        lin.forward_quantized(qx, sx)
        ev[3 * i + 2].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / args.steps
    quant_ms = sum(ev[3 * i].elapsed_time(ev[3 * i + 1]) for i in range(args.steps)) / args.steps
    gemm_ms = sum(ev[3 * i + 1].elapsed_time(ev[3 * i + 2]) for i in range(args.steps)) / args.steps
    flops = wl.linear_flops(M, N, K)
    gemm_tflops = flops / (gemm_ms * 1e-3) / 1e12
    traffic, counters = _profile_fields()
    line = {
        "metric": METRIC, "value": round(flops / (ms_step * 1e-3) / 1e12, 2), "unit": "TFLOP/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "e4m3 (fp32 accumulate)",
        "data": "synthetic (seeded N(0,1) activations with 0.1% outlier channels x20, N(0,0.02) weights)",
        "config": {"workload": "DiT QKV projection: quantize X + fp8 GEMM + bias", "M": M, "N": N, "K": K,
                   "seed": 2, "inputs_sha256_ok": inputs_ok, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "mfma", "achieved": round(gemm_tflops, 1), "peak": PEAK_FP8_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(gemm_tflops / PEAK_FP8_TFLOPS, 4), "traffic": traffic,
                     "kernel": "k_gemm_fp8 (EPI none, bias)", "kernel_ms": round(gemm_ms, 4),
                     "counters": counters},
    }
    extra = {"quantize_rows": {"ms": round(quant_ms, 4),
                               "GB/s": round(wl.quant_bytes(M, K) / (quant_ms * 1e-3) / 1e9, 1)}}
    extra["quantize_rows"]["frac_hbm"] = round(extra["quantize_rows"]["GB/s"] / PEAK_HBM_GBPS, 4)
    draws = None

    if not args.no_extra:
        reps = 10
        blk = wl.dit_block()
        x3, w3, b3 = wl.dit_ffn_up()
        (x4d, w4d), (x4o, w4o), g4 = wl.dit_ffn_down_attn_out()
        draws = dict(x2=x_cpu, w2=w_cpu, b2=b_cpu, x3=x3, w3=w3, b3=b3, x4d=x4d, w4d=w4d, x4o=x4o, w4o=w4o,
                     g4=g4, w5=blk["w0"], a5=blk["a"], b5=blk["b"], s5=blk["lora_scale"])
        # weight requantization, plain and with the fused rank-64 LoRA merge. A weight is
        # requantized once, so successive calls rotate over three copies (471 MB, more than
        # the 256 MB last-level cache): every call reads its weight from HBM.
        w0d, ad, bd = blk["w0"].to(dev), blk["a"].to(dev), blk["b"].to(dev)
        lscale = blk["lora_scale"]
        wcopies = [w0d, w0d.clone(), w0d.clone()]
        rot = itertools.cycle(wcopies)
        ms = _time_region(lambda: vdn_fp8.requantize_weight(next(rot)), reps)
        gbs = wl.requant_bytes(*w0d.shape) / (ms * 1e-3) / 1e9
        extra["requantize_weight"] = {"shape": list(w0d.shape), "ms": round(ms, 4), "GB/s": round(gbs, 1),
                                      "frac_hbm": round(gbs / PEAK_HBM_GBPS, 4)}
        ms = _time_region(lambda: vdn_fp8.requantize_weight(next(rot), lora=(ad, bd, lscale)), reps)
        del wcopies, rot
        gbs = wl.requant_bytes(*w0d.shape, rank=ad.shape[0]) / (ms * 1e-3) / 1e9
        extra["lora_merge_requantize"] = {"shape": list(w0d.shape), "rank": ad.shape[0], "ms": round(ms, 4),
                                          "GB/s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBPS, 4)}
        # one DiT block's four linears on the LoRA workload's own input (seed 5): the QKV
        # weight with its LoRA merged, attention-out + gate, FFN-up + GELU, FFN-down + gate
        # (the GELU applied by the FFN-down input's quantizer, gelu_quantize: the same codes
        # as the FFN-up GEMM's GELU epilogue followed by quantize_rows)
        qkv = _make_linear(blk["w0"], blk["qkv_bias"], dev, lora=(ad, bd, lscale))
        out_l = _make_linear(blk["w_out"], None, dev)
        up_l = _make_linear(blk["w_up"], blk["b_up"], dev)
        dn_l = _make_linear(blk["w_down"], None, dev)
        gate_d = blk["gate"].to(dev)
        x5 = blk["x"].to(dev)

        def block():
            qx, sx = vdn_fp8.quantize_rows(x5)
            qkv.forward_quantized(qx, sx)
            qx, sx = vdn_fp8.quantize_rows(x5)
            out_l.forward_quantized(qx, sx, epilogue="gate", gate=gate_d)
            qx, sx = vdn_fp8.quantize_rows(x5)
            hh = up_l.forward_quantized(qx, sx)
            qh, sh = vdn_fp8.gelu_quantize(hh)
            dn_l.forward_quantized(qh, sh, epilogue="gate", gate=gate_d)

        block()
        extra["block_linears"] = {"ms": round(_time_region(block, reps), 4),
                                  "flop": wl.linear_flops(M, 3 * 5120 + 5120 + 13824, 5120)
                                  + wl.linear_flops(M, 5120, 13824), "input": "dit_lora X (seed 5)"}
        del x5
        # the other linears on their own configs' inputs
        q3, s3 = vdn_fp8.quantize_rows(x3.to(dev))
        q4d, s4d = vdn_fp8.quantize_rows(x4d.to(dev))
        q4o, s4o = vdn_fp8.quantize_rows(x4o.to(dev))
        up3 = _make_linear(w3, b3, dev)
        dn4 = _make_linear(w4d, None, dev)
        out4 = _make_linear(w4o, None, dev)
        g4d = g4.to(dev)
        for name, fn, n_, k_ in (
                ("gemm_attn_out_gate", lambda: out4.forward_quantized(q4o, s4o, epilogue="gate", gate=g4d), 5120, 5120),
                ("gemm_ffn_up_gelu", lambda: up3.forward_quantized(q3, s3, epilogue="gelu_tanh"), 13824, 5120),
                ("gemm_ffn_down_gate", lambda: dn4.forward_quantized(q4d, s4d, epilogue="gate", gate=g4d), 5120, 13824)):
            ms = _time_region(fn, reps)
            tf = wl.linear_flops(M, n_, k_) / (ms * 1e-3) / 1e12
            extra[name] = {"ms": round(ms, 4), "TFLOP/s": round(tf, 1), "frac": round(tf / PEAK_FP8_TFLOPS, 4)}
        x4d_dev = x4d.to(dev)
        ms = _time_region(lambda: vdn_fp8.quantize_rows(x4d_dev), reps)
        gbs = wl.quant_bytes(M, 13824) / (ms * 1e-3) / 1e9
        extra["quantize_rows_13824"] = {"ms": round(ms, 4), "GB/s": round(gbs, 1),
                                        "frac_hbm": round(gbs / PEAK_HBM_GBPS, 4)}
        # the same rows through GELU(tanh) first (the DiT block's FFN-down input)
        ms = _time_region(lambda: vdn_fp8.gelu_quantize(x4d_dev), reps)
        gbs = wl.quant_bytes(M, 13824) / (ms * 1e-3) / 1e9
        extra["gelu_quantize_13824"] = {"ms": round(ms, 4), "GB/s": round(gbs, 1),
                                        "frac_hbm": round(gbs / PEAK_HBM_GBPS, 4)}
        del q3, q4d, q4o, up3, dn4, out4, x4d_dev
        # The QKV GEMM again with every code of X and W set to e4m3 1.0: same instructions, same
        # memory traffic, but operands that toggle no multiplier bits. The gap to the line above
        # is what random operands cost in clock (the part holds 2.4 GHz only on such data).
        lin_u = _make_linear(w_cpu, b_cpu, dev)
        lin_u.weight_fp8.view(torch.uint8).fill_(0x38)
        qx0, sx0 = vdn_fp8.quantize_rows(x)
        qu = torch.full_like(qx0.view(torch.uint8), 0x38).view(qx0.dtype)
        ms = _time_region(lambda: lin_u.forward_quantized(qu, sx0), reps)
        tf = flops / (ms * 1e-3) / 1e12
        extra["gemm_qkv_uniform_codes"] = {"ms": round(ms, 4), "TFLOP/s": round(tf, 1),
                                           "frac": round(tf / PEAK_FP8_TFLOPS, 4),
                                           "under_load": _under_load(lambda: lin_u.forward_quantized(qu, sx0))}
        extra["gemm_qkv_under_load"] = _under_load(lambda: lin.forward_quantized(qx0, sx0))
        del lin_u, qu
        # the bare MFMA loop on the same codes: the matrix cores' own rate on this data
        probe = _probe_lib()
        if probe is not None:
            cus = torch.cuda.get_device_properties(dev).multi_processor_count
            tiles_m, tiles_n = (M + 255) // 256, (N + 255) // 256
            blocks = (tiles_m * tiles_n + cus - 1) // cus * (K // 128)     # the GEMM's K blocks per CU
            ceil = _mfma_ceiling(probe, qx0.view(torch.uint8), lin.weight_fp8.view(torch.uint8), blocks, cus, reps)
            rnd = ceil["random_codes"]["TFLOP/s"]
            ceil["gemm_of_mfma_ceiling"] = round(gemm_tflops / rnd, 4)
            extra["mfma_random_ceiling"] = ceil
            line["roofline"]["of_mfma_ceiling"] = round(gemm_tflops / rnd, 4)
        # the reference's own forward_quantized on the same codes: torch._scaled_mm with the
        # rowwise scales (hipBLASLt here), then the bf16 bias add (fp8_linear.py:272-276)
        try:
            def ref_mm():
                return torch._scaled_mm(qx0, lin.weight_fp8.t(), scale_a=sx0, scale_b=lin.weight_scale,
                                        out_dtype=torch.bfloat16, use_fast_accum=True)
            ref_mm()
            torch.cuda.synchronize()
            ms_mm = _time_region(ref_mm, reps)
            ms_all = _time_region(lambda: ref_mm() + lin.bias, reps)
            tf = flops / (ms_all * 1e-3) / 1e12
            extra["torch_scaled_mm_qkv"] = {
                "call": "torch._scaled_mm(x_fp8, weight_fp8.t(), scale_a=[M,1], scale_b=[1,N], "
                        "out_dtype=bf16, use_fast_accum=True) + bias",
                "ms": round(ms_all, 4), "scaled_mm_ms": round(ms_mm, 4), "TFLOP/s": round(tf, 1),
                "frac": round(tf / PEAK_FP8_TFLOPS, 4), "ours_ms": round(gemm_ms, 4),
                "ours_over_torch": round(ms_all / gemm_ms, 4)}
        except RuntimeError as e:
            extra["torch_scaled_mm_qkv"] = {"error": str(e).splitlines()[0][:300]}
        # the H3 model's widths at one rank's share of a sequence (13107 tokens): fused QKV
        # [21504 x 5376] + bias, FF projection [28672 x 5376] + bias, FF down [5376 x 14336]
        # with the block's gate table and residual
        gh = torch.Generator().manual_seed(13)
        Mh = 13107
        xh = torch.randn(Mh, 5376, generator=gh).to(torch.bfloat16).to(dev)
        qxh, sxh = vdn_fp8.quantize_rows(xh)
        for name, n_, k_ in (("gemm_h3_qkv", 21504, 5376), ("gemm_h3_ff_proj", 28672, 5376)):
            wh = (0.02 * torch.randn(n_, k_, generator=gh)).to(torch.bfloat16)
            bh = (0.01 * torch.randn(n_, generator=gh)).to(torch.bfloat16)
            lh = _make_linear(wh, bh, dev)
            ms = _time_region(lambda: lh.forward_quantized(qxh, sxh), reps)
            tf = wl.linear_flops(Mh, n_, k_) / (ms * 1e-3) / 1e12
            extra[name] = {"shape": [Mh, n_, k_], "ms": round(ms, 4), "TFLOP/s": round(tf, 1),
                           "frac": round(tf / PEAK_FP8_TFLOPS, 4)}
            del lh
        hh3 = torch.randn(Mh, 14336, generator=gh).to(torch.bfloat16).to(dev)
        qh3, sh3 = vdn_fp8.quantize_rows(hh3)
        ld = _make_linear((0.02 * torch.randn(5376, 14336, generator=gh)).to(torch.bfloat16), None, dev)
        gt = (2 * torch.rand(4, 5376, generator=gh)).to(torch.bfloat16).to(dev)
        gix = torch.randint(0, 4, (Mh,), generator=gh).to(torch.int32).to(dev)
        ms = _time_region(lambda: ld.forward_quantized(qh3, sh3, epilogue="gate", gate=gt, gate_index=gix,
                                                       residual=xh), reps)
        tf = wl.linear_flops(Mh, 5376, 14336) / (ms * 1e-3) / 1e12
        extra["gemm_h3_ff_down_gate_residual"] = {"shape": [Mh, 5376, 14336], "ms": round(ms, 4),
                                                  "TFLOP/s": round(tf, 1), "frac": round(tf / PEAK_FP8_TFLOPS, 4)}
        ms = _time_region(lambda: ld.forward_quantized(qh3, sh3), reps)
        extra["gemm_h3_ff_down"] = {"shape": [Mh, 5376, 14336], "ms": round(ms, 4),
                                    "TFLOP/s": round(wl.linear_flops(Mh, 5376, 14336) / (ms * 1e-3) / 1e12, 1)}
        # the H3 FF sub-layer of fast_block_forward, per rank: fused (pre-norm + quantize,
        # projection GEMM, SwiGLU + quantize, down GEMM with the gate table and residual) vs
        # the same kernels with every stretch written out in bf16 (pre, quantize, GEMM,
        # swiglu + quantize, GEMM, post)
        from vdn_fp8 import fused_block as FB
        lp = _make_linear((0.02 * torch.randn(28672, 5376, generator=gh)).to(torch.bfloat16),
                          (0.01 * torch.randn(28672, generator=gh)).to(torch.bfloat16), dev)
        nw = (1 + 0.05 * torch.randn(5376, generator=gh)).to(torch.bfloat16).to(dev)
        tsc = (0.2 * torch.randn(4, 5376, generator=gh)).to(torch.bfloat16).to(dev)
        tsh = (0.2 * torch.randn(4, 5376, generator=gh)).to(torch.bfloat16).to(dev)

        def ff_fused():
            yq, ys = FB.pre_quantize(xh, nw, 1e-6, tsc, tsh, gix)
            a, s_ = vdn_fp8.swiglu_quantize(lp.forward_quantized(yq, ys))
            return ld.forward_quantized(a, s_, epilogue="gate", gate=gt, gate_index=gix, residual=xh)

        def ff_unfused():
            n_ = FB.pre(xh, nw, 1e-6, tsc, tsh, gix)
            a, s_ = vdn_fp8.swiglu_quantize(lp.forward_quantized(*vdn_fp8.quantize_rows(n_)))
            return FB.post(xh, gt, gix, ld.forward_quantized(a, s_))

        t_f, t_u = _time_pair(ff_fused, ff_unfused, reps)
        extra["ff_sublayer_h3"] = {"tokens": Mh, "fused_ms": round(t_f, 4), "unfused_ms": round(t_u, 4)}
        del ld, lp, hh3, qh3, xh, qxh
        # SwiGLU + quantize at the H3 FFN width (projection output [M, 2 x 14336])
        hh = torch.empty(M, 2 * 14336, dtype=torch.bfloat16, device=dev).normal_()
        ms = _time_region(lambda: vdn_fp8.swiglu_quantize(hh), reps)
        sw_bytes = M * (2 * 2 * 14336 + 14336 + 4)
        extra["swiglu_quantize_h3"] = {"shape": [M, 2 * 14336], "ms": round(ms, 4),
                                       "GB/s": round(sw_bytes / (ms * 1e-3) / 1e9, 1),
                                       "frac_hbm": round(sw_bytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)}
        del hh
        # the block's pre-norm (RMSNorm + AdaLN affine) fused with the quantizer: one table row
        # per latent frame (21 frames of 30 x 52 tokens), the rows chosen per token
        g = torch.Generator().manual_seed(6)
        frames = 21
        nw = (1 + 0.05 * torch.randn(K, generator=g)).to(torch.bfloat16).to(dev)
        nsc = (0.2 * torch.randn(frames, K, generator=g)).to(torch.bfloat16).to(dev)
        nsh = (0.2 * torch.randn(frames, K, generator=g)).to(torch.bfloat16).to(dev)
        nidx = (torch.arange(M) * frames // M).to(torch.int32).to(dev)
        ms = _time_region(lambda: vdn_fp8.pre_quantize(x, nw, 1e-6, nsc, nsh, nidx), reps)
        gbs = wl.quant_bytes(M, K) / (ms * 1e-3) / 1e9
        extra["pre_norm_quantize"] = {"ms": round(ms, 4), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBPS, 4)}
        # the same at the H3 width (one rank's 13107 tokens of hidden 5376, 5 frames)
        Mh3, Kh3, fh3 = 13107, 5376, 5
        xh3 = torch.randn(Mh3, Kh3, generator=g).to(torch.bfloat16).to(dev)
        nw3 = (1 + 0.05 * torch.randn(Kh3, generator=g)).to(torch.bfloat16).to(dev)
        nsc3 = (0.2 * torch.randn(fh3, Kh3, generator=g)).to(torch.bfloat16).to(dev)
        nsh3 = (0.2 * torch.randn(fh3, Kh3, generator=g)).to(torch.bfloat16).to(dev)
        nidx3 = (torch.arange(Mh3) * fh3 // Mh3).to(torch.int32).to(dev)
        ms = _time_region(lambda: vdn_fp8.pre_quantize(xh3, nw3, 1e-6, nsc3, nsh3, nidx3), reps)
        gbs = wl.quant_bytes(Mh3, Kh3) / (ms * 1e-3) / 1e9
        extra["pre_norm_quantize_h3"] = {"shape": [Mh3, Kh3], "ms": round(ms, 4), "GB/s": round(gbs, 1),
                                         "frac_hbm": round(gbs / PEAK_HBM_GBPS, 4)}
        del xh3
        # the block's gated residual add (`post`) over [M, 5120] with a 2-row gate table
        br_ = torch.randn(M, K, device=dev).to(torch.bfloat16)
        gtab = (2 * torch.rand(2, K, device=dev)).to(torch.bfloat16)
        gid = torch.randint(0, 2, (M,), device=dev)
        ms = _time_region(lambda: FB.post(x, gtab, gid, br_), reps)
        gbs = 3 * M * K * 2 / (ms * 1e-3) / 1e9
        extra["post_gated_residual"] = {"shape": [M, K], "ms": round(ms, 4), "GB/s": round(gbs, 1),
                                        "frac_hbm": round(gbs / PEAK_HBM_GBPS, 4)}
        del br_
        # QK-norm + rope on q of the QKV output (40 heads of 128, a strided view of the fused
        # [M, 3 x 5120] projection output), fp32 cos/sin tables [M, 128]
        qkv_out = lin.forward_quantized(*vdn_fp8.quantize_rows(x))
        qv = qkv_out[:, :5120].unflatten(-1, (40, 128))
        nq = (1 + 0.05 * torch.randn(128, generator=g)).to(torch.bfloat16).to(dev)
        th = torch.rand(M, 64, device=dev) * 6.28
        cs, sn = torch.cat([th.cos(), th.cos()], 1), torch.cat([th.sin(), th.sin()], 1)
        ms = _time_region(lambda: vdn_fp8.qk_prep(qv, nq, 1e-6, cs, sn), reps)
        qk_bytes = M * 5120 * 2 * 2 + 2 * M * 128 * 4
        gbs = qk_bytes / (ms * 1e-3) / 1e9
        extra["qk_prep_q"] = {"shape": [M, 40, 128], "ms": round(ms, 4), "GB/s": round(gbs, 1),
                              "frac_hbm": round(gbs / PEAK_HBM_GBPS, 4)}
        del qkv_out, qv
        # each HBM-bound kernel against a bare stream of its own read and write bytes, and
        # against a torch library kernel with the same read : write mix
        probe = _probe_lib()
        nw_, kw_ = extra["requantize_weight"]["shape"]
        mixes = {   # names: (read bytes, write bytes, non-temporal stores, source copies rotated)
            ("quantize_rows", "pre_norm_quantize"): (2 * M * K, M * K + 4 * M, False, 1),
            ("pre_norm_quantize_h3",): (2 * 13107 * 5376, 13107 * 5376 + 4 * 13107, False, 1),
            ("requantize_weight", "lora_merge_requantize"): (2 * nw_ * kw_, nw_ * kw_ + 4 * nw_, False, 3),
            ("quantize_rows_13824", "gelu_quantize_13824"): (2 * M * 13824, M * 13824 + 4 * M, M * 13824 >= (256 << 20), 1),
            ("swiglu_quantize_h3",): (4 * M * 14336, M * 14336 + 4 * M, True, 1),
            ("post_gated_residual",): (2 * M * K * 2, M * K * 2, True, 1),
            ("qk_prep_q",): (M * 5120 * 2, M * 5120 * 2, True, 1),
        }
        if probe is not None:
            src = torch.empty(1900 << 20, dtype=torch.uint8, device=dev).fill_(1)
            dst = torch.empty(460 << 20, dtype=torch.uint8, device=dev)
            rate = functools.partial(_stream_rate, probe, src, dst)
            for names, (rb_, wb_, nt_, rot_) in mixes.items():
                gbs = rate(rb_, wb_, nt_, rotate=rot_)
                for n_ in names:
                    if n_ in extra and "GB/s" in extra[n_]:
                        extra[n_]["stream_GB/s"] = round(gbs, 1)
                        extra[n_]["of_stream"] = round(extra[n_]["GB/s"] / gbs, 4)
            del src, dst
        for names, (rb_, wb_, _, rot_) in mixes.items():
            gbs = _torch_rate(rb_, wb_, rotate=rot_)
            for n_ in names:
                if n_ in extra and "GB/s" in extra[n_]:
                    extra[n_]["torch_GB/s"] = round(gbs, 1)
                    extra[n_]["of_torch"] = round(extra[n_]["GB/s"] / gbs, 4)
        extra["torch_kernels"] = ("copy_ (1:1), torch.add(a, b, out=c) (2:1), torch.sum over groups of four (4:1), "
                                  "bf16, the same bytes as each kernel")
        extra["gpu_clock"] = _gpu_clock()
    line["extra"] = extra
    if not args.no_cpu_baseline:
        if draws is None:
            blk = wl.dit_block()
            x3, w3, b3 = wl.dit_ffn_up()
            (x4d, w4d), (x4o, w4o), g4 = wl.dit_ffn_down_attn_out()
            draws = dict(x2=x_cpu, w2=w_cpu, b2=b_cpu, x3=x3, w3=w3, b3=b3, x4d=x4d, w4d=w4d, x4o=x4o,
                         w4o=w4o, g4=g4, w5=blk["w0"], a5=blk["a"], b5=blk["b"], s5=blk["lora_scale"])
        import numpy as np
        u16 = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)
        draws = {k: (u16(v) if isinstance(v, torch.Tensor) else v) for k, v in draws.items()}
        line["cpu_baseline"] = cpu_baseline(draws)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
