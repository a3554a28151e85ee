"""Benchmark of the W8A8 linear family on one MI355X.

Default workload ("step"): one pass of the Qwen-Image-style DiT block's linear
set at 1600x896 with CFG, M = 2 x (5600 + 256) = 11712 tokens, hidden 3072:
  quantize -> QKV GEMM (N=9216), quantize -> out-proj (N=3072),
  quantize -> FFN-up GEMM (N=12288, GELU-tanh fused epilogue),
  quantize -> FFN-down GEMM (K=12288, N=3072).
Synthetic seeded inputs (bf16 N(0,1) activations, int8 U[-127,127] weights,
fp32 per-channel scales U(1e-3,1e-2), bf16 bias N(0,0.02)), resident in HBM;
4 sets of the step's three inputs rotate from step to step (864 MB, beyond the
256 MB Infinity Cache).  After the timed steps the last step's FFN outputs are
checked on sampled rows against a float64 recomputation ("output_check").
value = GEMM TOPS of the whole step (2*M*N*K summed over the 4 linears,
divided by the step time, quantization included in the time).  The default
50 warmup steps cover the clock settling of a loaded MI355X: measured step
by step, the first ~25 steps of the set run up to 40% slower (the first few
launches meet the power limit's transient), after which the step time holds
within 0.3% over hundreds of steps; the 100 timed steps then take ~0.13 s.

Also measured and reported beside it: per-linear TOPS, the per-token
quantizer's GB/s (M=11712, K=3072 and K=12288), the adaLN GEMV's GB/s
(M=2, K=3072, N=18432), and fused vs unfused quant+GEMM on the outlier
workload (M=11712, K=3072, N=12288, Student-t(3) activations), the block
glue's GB/s (adaLN, gated residual at 2x5856x3072; QK RMSNorm + RoPE on q / k
views into a 2x5856x3x24x128 QKV output), and the 60-block DiT denoising step
at M=19904 (ms/step, W8A8 and glue shares; attention in torch).  The memory-bound kernels rotate through enough
buffer sets to exceed the 256 MB Infinity Cache so they measure HBM, not cache.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--only KERNEL] [--no-cpu] [--no-dit-step]
"""
import argparse
import json
import os
import statistics
import subprocess
import sys
import time

import torch

PEAK_INT8_TOPS = 5000.0       # MI355X dense INT8 MFMA, TOPS
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E, GB/s
M_TOK = 2 * (5600 + 256)      # 11712
HID, FFN, QKV = 3072, 12288, 9216
N_SETS = 4                    # rotating input sets of the step
LINEARS = [("qkv", HID, QKV, False), ("out", HID, HID, False), ("up", HID, FFN, True),
           ("down", FFN, HID, False)]  # (name, K, N, gelu epilogue)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=50)
    p.add_argument("--only", default=None,
                   help="run only one kernel in a loop (for rocprofv3 counters): "
                        "up_gemm | quant | quant12288 | gemv | convrot_quant | rms_rope | step | copy | dit_step")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-dit-step", action="store_true", help="skip the 60-block DiT step extra")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    return p.parse_args()


def gen(seed):
    return torch.Generator().manual_seed(seed)


def make_linear(k, n, seed, dev):
    g = gen(seed)
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    ws = torch.rand(n, generator=g) * 9e-3 + 1e-3
    b = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
    return w.to(dev), ws.to(dev), b.to(dev)


def student_t(m, k, seed):
    g = gen(seed)
    z = torch.randn(m, k, generator=g)
    chi = torch.randn(m, k, 3, generator=g).pow(2).sum(-1)
    x = z / torch.sqrt(chi / 3.0)
    idx = torch.randperm(k, generator=g)[: max(1, k // 1000)]
    x[:, idx] *= 50.0
    return x.to(torch.bfloat16)


class Timer:
    """HIP events on torch's current stream (the stream every W8A8 kernel is
    launched on): per-launch durations of one kernel inside the timed region."""

    def __init__(self):
        self.pairs = []

    def start(self):
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        return e

    def stop(self, s):
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        self.pairs.append((s, e))

    def mean_ms(self):
        return statistics.fmean(s.elapsed_time(e) for s, e in self.pairs)


def median_of_batches(fn, warmup=20, batches=7, calls=30):
    """The reference's timing method: 20 warmups, 7 batches x 30 calls,
    median of batch means (experiments/.../INT8-KITCHEN.md:35-39)."""
    for _ in range(warmup):
        fn(0)
    torch.cuda.synchronize()
    means = []
    i = 0
    for _ in range(batches):
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(calls):
            fn(i)
            i += 1
        e.record()
        torch.cuda.synchronize()
        means.append(s.elapsed_time(e) / calls)
    return statistics.median(means)


def host_cpu():
    """nproc and the lscpu model / core / thread counts of the host."""
    info = {"nproc": os.cpu_count()}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        keys = {"Model name": "model", "CPU(s)": "cpus", "Thread(s) per core": "threads_per_core",
                "Core(s) per socket": "cores_per_socket", "Socket(s)": "sockets"}
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in keys:
                info[keys[k.strip()]] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return info


def cpu_time_per_call(fn, warmup=20, batches=7, calls=30):
    """The reference's method on the host: 20 warmups, 7 batches x 30 calls,
    median of batch means (experiments/.../INT8-KITCHEN.md:35-39); seconds."""
    for _ in range(warmup):
        fn()
    means = []
    for _ in range(batches):
        t0 = time.perf_counter()
        for _ in range(calls):
            fn()
        means.append((time.perf_counter() - t0) / calls)
    return statistics.median(means)


def cpu_baseline(seconds):
    """The reference's LibTorch-CPU route (oracle/torch_eager.py, same ATen op
    sequence as inference/src/int8_linear.rs:198-277), timed on the host's
    cores: the headline value on a bounded sample of the bench's workload (the
    4 block linears at M=256 rows, repeated for ~`seconds`), and the two
    CPU-sized configurations with the reference's timing method: the single
    linear M=256 K=3072 N=3072 and the adaLN GEMV M=2 K=3072 N=18432."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import torch_eager as TE
    torch.set_num_threads(os.cpu_count() or 1)
    m = 256
    ops_per_pass = 0
    layers = []
    for i, (name, k, n, gelu) in enumerate(LINEARS):
        w, ws, b = make_linear(k, n, 100 + i, "cpu")
        x = torch.randn(m, k, generator=gen(200 + i)).to(torch.bfloat16)
        layers.append((x, w, ws, b))
        ops_per_pass += 2 * m * k * n
    def one_pass():
        for x, w, ws, b in layers:
            TE.int8_linear(x, w, ws, b, torch.bfloat16)
    one_pass()  # warmup
    t0 = time.perf_counter()
    passes = 0
    while True:
        one_pass()
        passes += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    tops = ops_per_pass * passes / el / 1e12
    host = host_cpu()

    # the two CPU configurations, 20 warmups + 7 x 30 calls each
    k, n = 3072, 3072
    w, ws, b = make_linear(k, n, 300, "cpu")
    x = torch.randn(256, k, generator=gen(301)).to(torch.bfloat16)
    t_c1 = cpu_time_per_call(lambda: TE.int8_linear(x, w, ws, b, torch.bfloat16))
    k, n = 3072, 18432
    w2, ws2, b2 = make_linear(k, n, 302, "cpu")
    x2 = torch.randn(2, k, generator=gen(303)).to(torch.bfloat16)
    t_c2 = cpu_time_per_call(lambda: TE.int8_linear(x2, w2, ws2, b2, torch.bfloat16))
    gemv_bytes = n * k + 2 * k * 2 + 2 * n * 2 + n * 4   # weights, x, out, scales
    return {"value": round(tops, 4), "unit": "TOPS", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"block linear set (QKV, out, up, down) at M=256 tokens, {passes} passes "
                      f"in {el:.1f} s, LibTorch CPU int8_linear op sequence; host {host.get('model', '')}",
            "host": host,
            "single_linear_M256_K3072_N3072": {"ms": round(t_c1 * 1e3, 3),
                                               "TOPS": round(2 * 256 * 3072 * 3072 / t_c1 / 1e12, 4),
                                               "method": "20 warmups, median of 7 x 30 calls"},
            "adaln_gemv_M2_K3072_N18432": {"ms": round(t_c2 * 1e3, 3),
                                           "GB/s": round(gemv_bytes / t_c2 / 1e9, 2),
                                           "method": "20 warmups, median of 7 x 30 calls"}}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    import imagine_amd as W
    W._lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    print(f"[bench] device {torch.cuda.get_device_name(0)}", file=sys.stderr, flush=True)

    # ---- block linear set operands
    layers = []
    for i, (name, k, n, gelu) in enumerate(LINEARS):
        w, ws, b = make_linear(k, n, 10 + i, dev)
        layers.append((name, k, n, gelu, w, ws, b))
    # N_SETS input sets (3 x 72 MB each) rotate from step to step, so the
    # quantizers read their rows from HBM, not from the 256 MB Infinity Cache.
    xsets = [[torch.randn(M_TOK, HID, device=dev, generator=torch.Generator(device=dev).manual_seed(3 * i + j + 1))
              .to(torch.bfloat16) for j in range(3)] for i in range(N_SETS)]
    x_ffn = xsets[0][2]
    qbuf = {k: torch.empty((M_TOK, k), dtype=torch.int8, device=dev) for k in (HID, FFN)}
    sbuf = torch.empty((M_TOK, 1), dtype=torch.float32, device=dev)
    outs = {name: torch.empty((M_TOK, n), dtype=torch.bfloat16, device=dev) for name, _, n, *_ in layers}
    lib = W._lib.load()
    stream = lambda: torch.cuda.current_stream().cuda_stream

    def quant(x, q):
        W._lib.check(lib.w8a8_quantize_rowwise(x.data_ptr(), W._lib.BF16, q.data_ptr(), sbuf.data_ptr(),
                                               x.shape[0], x.shape[1], 0, stream()))

    def gemm(q, layer, out, gelu):
        name, k, n, _, w, ws, b = layer
        W._lib.check(lib.w8a8_gemm_dequant(q.data_ptr(), w.data_ptr(), sbuf.data_ptr(), ws.data_ptr(), n,
                                           b.data_ptr(), out.data_ptr(), W._lib.BF16, M_TOK, n, k,
                                           W._lib.ACT_GELU_TANH if gelu else 0, stream()))

    up_timer = Timer()

    nstep = [0]

    def step(timed=False):
        xq, xo, xf = xsets[nstep[0] % N_SETS]
        nstep[0] += 1
        quant(xq, qbuf[HID]); gemm(qbuf[HID], layers[0], outs["qkv"], False)
        quant(xo, qbuf[HID]); gemm(qbuf[HID], layers[1], outs["out"], False)
        quant(xf, qbuf[HID])
        s = up_timer.start() if timed else None
        gemm(qbuf[HID], layers[2], outs["up"], True)
        if timed:
            up_timer.stop(s)
        quant(outs["up"], qbuf[FFN]); gemm(qbuf[FFN], layers[3], outs["down"], False)

    if args.only == "dit_step":
        print(json.dumps(measure_dit_step(W, dev, steps=max(args.steps, 1), warmup=args.warmup)), flush=True)
        return
    if args.only:
        run_only(args, W, lib, dev, layers, step, quant, gemm, qbuf, x_ffn, outs)
        return

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(timed=True)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps
    step_ops = sum(2 * M_TOK * k * n for _, k, n, *_ in LINEARS)
    value = step_ops / (ms_per_step * 1e-3) / 1e12
    up_ops = 2 * M_TOK * HID * FFN
    up_ms = up_timer.mean_ms()
    up_tops = up_ops / (up_ms * 1e-3) / 1e12
    print(f"[bench] step {ms_per_step:.3f} ms -> {value:.1f} TOPS; up GEMM {up_ms*1e3:.1f} us "
          f"-> {up_tops:.1f} TOPS", file=sys.stderr, flush=True)

    check = validate_step(layers, xsets[(nstep[0] - 1) % N_SETS][2], qbuf, sbuf, outs)
    print(f"[bench] outputs of the last timed step: {check}", file=sys.stderr, flush=True)

    extras = measure_extras(W, lib, dev, layers, quant, gemm, qbuf, sbuf, outs, xsets[0])
    if not args.no_dit_step:
        extras["dit_step_60_blocks_M19904"] = measure_dit_step(W, dev)
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)
    line = {
        "metric": "W8A8 GEMM TOPS (% INT8 MFMA peak) at Qwen-DiT 1600x896 shapes; quant GB/s",
        "value": round(value, 2), "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "qwen_dit_block_linear_set_1600x896_cfg", "M": M_TOK, "hidden": HID,
                   "ffn": FFN, "linears": "qkv 3072->9216, out 3072->3072, up 3072->12288 +gelu_tanh, "
                                         "down 12288->3072; per-token quant of each input included",
                   "parallelism": "single_gpu", "pct_int8_peak": round(100 * value / PEAK_INT8_TOPS, 2)},
        "roofline": {"kernel": "gemm_mfma_dma DmaCfg<256,256,128,64,128,2,2> (FFN-up 11712x3072x12288, "
                               "bf16 out, GELU epilogue)",
                     "bound": "mfma", "achieved": round(up_tops, 2), "peak": PEAK_INT8_TOPS,
                     "unit": "TOPS", "frac": round(up_tops / PEAK_INT8_TOPS, 4), "traffic": traffic_bytes(),
                     "launch_us": round(up_ms * 1e3, 2), "algorithmic_ops": up_ops},
        "cpu_baseline": cpu,
        "output_check": check,
        "extras": extras,
    }
    print(json.dumps(line), flush=True)


def validate_step(layers, x_ffn, qbuf, sbuf, outs, nrows=8):
    """Sanity check of the last timed step's FFN outputs (sampled rows) against
    a float64 torch recomputation from the int8 codes those GEMMs consumed:
    FFN-up from the codes of x_ffn (its per-token scales amax/127 recomputed
    from x_ffn), FFN-down from the codes and scales of the FFN-up output.  Not
    the parity tests (those hold every value bit for bit against the oracle);
    the bound is the north star's max relative error 1e-2."""
    rows = torch.linspace(0, M_TOK - 1, nrows, device=x_ffn.device).long()
    _, _, _, _, w_up, ws_up, b_up = layers[2]
    _, _, _, _, w_dn, ws_dn, b_dn = layers[3]
    xf = x_ffn[rows].double()
    s_in = (xf.abs().amax(dim=1).float() / 127.0).clamp_min(1e-30).double()
    acc_up = qbuf[HID][rows].double() @ w_up.double().t()
    lin = acc_up * s_in[:, None] * ws_up.double() + b_up.double()
    up_ref = 0.5 * lin * (1.0 + torch.tanh(0.7978845608028654 * (lin + 0.044715 * lin ** 3)))
    acc_dn = qbuf[FFN][rows].double() @ w_dn.double().t()
    dn_ref = acc_dn * sbuf[rows].double() * ws_dn.double() + b_dn.double()

    def rel(out, ref):
        return float(((out.double() - ref).abs().amax(dim=1) / ref.abs().amax(dim=1)).max())

    e_up, e_dn = rel(outs["up"][rows], up_ref), rel(outs["down"][rows], dn_ref)
    return {"rows": nrows, "ffn_up_max_rel_err": round(e_up, 6), "ffn_down_max_rel_err": round(e_dn, 6),
            "ok": e_up <= 1e-2 and e_dn <= 1e-2}


def traffic_bytes():
    """HBM bytes per launch of the roofline kernel, read from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary of the same kernel and workload
    (profiles/)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "hbm_traffic_ffn_up_gemm_and_quant_M11712.txt")
    key = "gemm_mfma_dma DmaCfg<256,256,128,64,128,2,2> ffn_up traffic_bytes_per_launch:"
    try:
        with open(path) as f:
            for line in f:
                if key in line:
                    return int(line.split(key, 1)[1].split()[0])
    except (OSError, ValueError):
        pass
    return None


def measure_extras(W, lib, dev, layers, quant, gemm, qbuf, sbuf, outs, x_in):
    ex = {}
    stream = lambda: torch.cuda.current_stream().cuda_stream
    # per-linear GEMM (no quant), reference timing method, each on the codes
    # and scales of its own input: FFN-down first, on the last step's
    # quantized FFN-up output, then QKV, out-proj and FFN-up, each after
    # quantizing its input
    own_input = {"qkv": x_in[0], "out": x_in[1], "up": x_in[2]}
    for layer in [layers[3]] + layers[:3]:
        name, k, n, gelu, *_ = layer
        if name in own_input:
            quant(own_input[name], qbuf[k])
        q = qbuf[k]
        ms = median_of_batches(lambda i: gemm(q, layer, outs[name], gelu), warmup=5, batches=5, calls=10)
        tops = 2 * M_TOK * k * n / (ms * 1e-3) / 1e12
        ex[f"gemm_{name}"] = {"us": round(ms * 1e3, 1), "TOPS": round(tops, 1),
                              "pct_peak": round(100 * tops / PEAK_INT8_TOPS, 1)}
    # quantizer GB/s, rotating input sets past the Infinity Cache
    for k in (HID, FFN):
        per = 2 * M_TOK * k + M_TOK * k + 4 * M_TOK
        nsets = max(2, int(1.2e9 // per) + 1)
        xs = [torch.randn(M_TOK, k, device=dev, dtype=torch.bfloat16) for _ in range(nsets)]
        qs = [torch.empty(M_TOK, k, dtype=torch.int8, device=dev) for _ in range(nsets)]
        ss = torch.empty(M_TOK, dtype=torch.float32, device=dev)
        def run(i):
            j = i % nsets
            W._lib.check(lib.w8a8_quantize_rowwise(xs[j].data_ptr(), W._lib.BF16, qs[j].data_ptr(),
                                                   ss.data_ptr(), M_TOK, k, 0, stream()))
        ms = median_of_batches(run)
        ex[f"quant_K{k}"] = {"us": round(ms * 1e3, 2), "GB/s": round(per / (ms * 1e-3) / 1e9, 1),
                             "pct_hbm_peak": round(100 * per / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 1),
                             "bytes": per, "buffer_sets": nsets}

        # ConvRot (Hadamard-256 rotation fused into the quantizer), same bytes
        def run_convrot(i):
            j = i % nsets
            W._lib.check(lib.w8a8_quantize_rowwise_convrot(xs[j].data_ptr(), W._lib.BF16, qs[j].data_ptr(),
                                                           ss.data_ptr(), M_TOK, k, 256, 0, None, 0, stream()))
        ms = median_of_batches(run_convrot)
        ex[f"convrot_quant_K{k}"] = {"us": round(ms * 1e3, 2), "GB/s": round(per / (ms * 1e-3) / 1e9, 1),
                                     "pct_hbm_peak": round(100 * per / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 1),
                                     "bytes": per, "buffer_sets": nsets}
        del xs, qs
    # adaLN GEMV, M=2 K=3072 N=18432, rotating weights
    m, k, n = 2, 3072, 18432
    per = n * k + 4 * n + 2 * m * k + 2 * m * n + 2 * n
    nsets = max(2, int(1.2e9 // per) + 1)
    ws_ = [torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev) for _ in range(nsets)]
    wsc = torch.rand(n, device=dev) * 9e-3 + 1e-3
    bias = (torch.randn(n, device=dev) * 0.02).to(torch.bfloat16)
    xsil = torch.nn.functional.silu(torch.randn(m, k, device=dev)).to(torch.bfloat16)
    q, xsc = W.quantize_rowwise(xsil)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
    def gemv(i):
        w = ws_[i % nsets]
        W._lib.check(lib.w8a8_gemv_dequant(q.data_ptr(), w.data_ptr(), xsc.data_ptr(), wsc.data_ptr(), n,
                                           bias.data_ptr(), out.data_ptr(), W._lib.BF16, m, n, k, 0, stream()))
    ms = median_of_batches(gemv)
    ex["gemv_adaln_M2_K3072_N18432"] = {"us": round(ms * 1e3, 2), "GB/s": round(per / (ms * 1e-3) / 1e9, 1),
                                        "pct_hbm_peak": round(100 * per / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 1),
                                        "bytes": per, "buffer_sets": nsets}
    del ws_
    # block glue at the DiT block's hidden states [2, 5856, 3072] bf16 (the
    # norm1/norm2 adaLN and the two gated residuals), rotating sets
    hb, ht = 2, M_TOK // 2
    hbytes = hb * ht * HID * 2
    per = 2 * hbytes                       # adaLN: read x, write out
    nsets = max(2, int(1.2e9 // per) + 1)
    hx = [torch.randn(hb, ht, HID, device=dev).to(torch.bfloat16) for _ in range(nsets)]
    ho = [torch.empty_like(hx[0]) for _ in range(nsets)]
    hs = (torch.randn(hb, 1, HID, device=dev) * 0.3).to(torch.bfloat16)
    hz = torch.zeros(hb, 1, HID, device=dev, dtype=torch.bfloat16)
    def adaln(i):
        j = i % nsets
        W._lib.check(lib.w8a8_adaln(hx[j].data_ptr(), hs.data_ptr(), hz.data_ptr(), ho[j].data_ptr(), hb * ht,
                                    HID, ht, ht, 1e-6, W._lib.BF16, 0, stream()))
    ms = median_of_batches(adaln)
    ex["adaln_2x5856x3072"] = {"us": round(ms * 1e3, 2), "GB/s": round(per / (ms * 1e-3) / 1e9, 1),
                               "pct_hbm_peak": round(100 * per / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 1),
                               "bytes": per, "buffer_sets": nsets}
    per = 3 * hbytes                       # gated residual: read x and y, write x
    def gres(i):
        j = i % nsets
        W._lib.check(lib.w8a8_gated_residual(hx[j].data_ptr(), ho[j].data_ptr(), hs.data_ptr(), hs.data_ptr(),
                                             hx[j].data_ptr(), hb, ht, HID, 256, W._lib.BF16, stream()))
    ms = median_of_batches(gres)
    ex["gated_residual_2x5856x3072"] = {"us": round(ms * 1e3, 2), "GB/s": round(per / (ms * 1e-3) / 1e9, 1),
                                        "pct_hbm_peak": round(100 * per / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 1),
                                        "bytes": per, "buffer_sets": nsets}
    del hx, ho
    # QK RMSNorm + RoPE on q and k read in place out of the fused QKV output
    # [2, 5856, 3, 24, 128] bf16, packed outputs; per launch: q and k read,
    # q_out and k_out written, the fp32 [5856, 64, 2, 2] rotation table read
    nh, hd = 24, HID // 24
    per = 4 * hbytes + ht * (hd // 2) * 16
    nsets = max(2, int(1.2e9 // (5 * hbytes)) + 1)
    qkv = [torch.randn(hb, ht, 3, nh, hd, device=dev).to(torch.bfloat16) for _ in range(nsets)]
    qo = [torch.empty(hb, ht, nh, hd, device=dev, dtype=torch.bfloat16) for _ in range(2 * nsets)]
    fr = torch.randn(ht, hd // 2, 2, 2, device=dev)
    sc = torch.ones(hd, device=dev, dtype=torch.bfloat16)
    def rope(i):
        j = i % nsets
        W._lib.check(lib.w8a8_rms_rope(qkv[j].data_ptr(), qkv[j][:, :, 1].data_ptr(), fr.data_ptr(), sc.data_ptr(),
                                       sc.data_ptr(), qo[2 * j].data_ptr(), qo[2 * j + 1].data_ptr(), hb, ht, nh, hd,
                                       3 * nh * hd, 0, 1e-6, W._lib.BF16, stream()))
    ms = median_of_batches(rope)
    ex["rms_rope_qkv_2x5856x24x128"] = {"us": round(ms * 1e3, 2), "GB/s": round(per / (ms * 1e-3) / 1e9, 1),
                                        "pct_hbm_peak": round(100 * per / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 1),
                                        "bytes": per, "buffer_sets": nsets}
    del qkv, qo
    # outlier workload: fused quant+GEMM vs unfused
    m, k, n = M_TOK, HID, FFN
    x = student_t(m, k, 3).to(dev)
    w, wsc, b = make_linear(k, n, 30, dev)
    qo = torch.empty(m, k, dtype=torch.int8, device=dev)
    so = torch.empty(m, 1, dtype=torch.float32, device=dev)
    o = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
    def unfused(i):
        W._lib.check(lib.w8a8_quantize_rowwise(x.data_ptr(), W._lib.BF16, qo.data_ptr(), so.data_ptr(), m, k, 0, stream()))
        W._lib.check(lib.w8a8_gemm_dequant(qo.data_ptr(), w.data_ptr(), so.data_ptr(), wsc.data_ptr(), n,
                                           b.data_ptr(), o.data_ptr(), W._lib.BF16, m, n, k, 0, stream()))
    def fused(i):
        W._lib.check(lib.w8a8_row_scales(x.data_ptr(), W._lib.BF16, so.data_ptr(), m, k, 0, stream()))
        W._lib.check(lib.w8a8_gemm_dequant_xq(x.data_ptr(), W._lib.BF16, so.data_ptr(), w.data_ptr(),
                                              wsc.data_ptr(), n, b.data_ptr(), o.data_ptr(), W._lib.BF16,
                                              m, n, k, 0, stream()))
    mu = median_of_batches(unfused, warmup=5, batches=5, calls=10)
    mf = median_of_batches(fused, warmup=5, batches=5, calls=10)
    ops = 2 * m * n * k
    ex["outlier_quant_gemm_11712x3072x12288"] = {
        "unfused_us": round(mu * 1e3, 1), "fused_us": round(mf * 1e3, 1),
        "unfused_TOPS": round(ops / (mu * 1e-3) / 1e12, 1), "fused_TOPS": round(ops / (mf * 1e-3) / 1e12, 1)}
    return ex


def measure_dit_step(W, dev, steps=2, warmup=1, blocks=60):
    """The 60-block Qwen-Image-style MMDiT denoising step: hidden 3072, 24 heads
    x 128, FFN 12288 (GELU-tanh), a 1600x896 latent (5600 tokens) + one 1 MP
    reference image (4096) + 256 text tokens, CFG batch 2 (M = 19904), on
    random-init int8 weights (60 distinct sets, ~6.8 GB, resident in HBM).
    Per block, as the reference's block forward (models/qwen_image21/dit.rs:
    285-340): text and image modulation GEMVs (M=2, N=18432) -> norm1
    (modulated_norm, text prefix 256) -> QKV -> QK RMSNorm + RoPE
    (imagine_amd.rms_rope; a 1D frequency table stands in for the 2D one) ->
    attention (torch fused SDPA; no math fallback) -> out-proj -> gated
    residual -> norm2 -> FFN-up -> FFN-down with input_act gelu_tanh -> gated
    residual.  norm1 and norm2 only feed QKV and FFN-up, so they run as the
    fused norm + quantizer (modulated_norm_quant, the same codes as norm then
    quantize) followed by the GEMM; the other linears go through
    imagine_amd.int8_linear (quantizer + GEMM/GEMV), the residuals through
    imagine_amd.glue.  HIP events around each library call inside the timed
    steps give the W8A8 (GEMM, GEMV, quantizer), fused norm + quantizer and
    glue shares."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    B, T_txt = 2, 256
    T = 5600 + 4096 + T_txt
    D, H, HD = HID, 24, 128
    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(4)

    def lin(k, n):
        w = torch.randint(-127, 128, (n, k), device=dev, dtype=torch.int8, generator=g)
        ws = torch.rand(n, device=dev, generator=g) * 9e-3 + 1e-3
        b = (torch.randn(n, device=dev, generator=g) * 0.02).to(bf)
        return w, ws, b

    blks = [{"mod_txt": lin(D, 6 * D), "mod_img": lin(D, 6 * D), "qkv": lin(D, 3 * D), "out": lin(D, D),
             "up": lin(D, FFN), "down": lin(FFN, D),
             "qn": (1 + 0.1 * torch.randn(HD, device=dev, generator=g)).to(bf),
             "kn": (1 + 0.1 * torch.randn(HD, device=dev, generator=g)).to(bf)} for _ in range(blocks)]
    temb = torch.nn.functional.silu(torch.randn(B, D, device=dev, generator=g)).to(bf)
    x0 = torch.randn(B, T, D, device=dev, generator=g).to(bf)
    inv = 1.0 / (10000.0 ** (torch.arange(0, HD, 2, device=dev).float() / HD))
    ang = torch.arange(T, device=dev).float()[:, None] * inv[None]
    c_, s_ = ang.cos(), ang.sin()
    freqs = torch.stack([torch.stack([c_, -s_], -1), torch.stack([s_, c_], -1)], -2)[None, :, None].contiguous()
    zero = torch.zeros(B, 1, D, device=dev, dtype=bf)
    ev = {"w8a8": [], "glue": [], "norm_quant": []}

    def timed(kind, fn, *a, **k):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        r = fn(*a, **k)
        e.record()
        ev[kind].append((s, e))
        return r

    def block(x, p):
        mt = [c.reshape(B, 1, D).contiguous() for c in timed("w8a8", W.int8_linear, temb, *p["mod_txt"]).chunk(6, -1)]
        mi = [c.reshape(B, 1, D).contiguous() for c in timed("w8a8", W.int8_linear, temb, *p["mod_img"]).chunk(6, -1)]
        q1, s1 = timed("norm_quant", W.modulated_norm_quant, x, (mt[1], mi[1]), T_txt, zero, 1e-6)
        qkv = timed("w8a8", W.gemm_dequant, q1, p["qkv"][0], s1, *p["qkv"][1:], torch.bfloat16)
        qkv = qkv.view(B, T, 3, H, HD)
        q, k = timed("glue", W.rms_rope, qkv[:, :, 0], qkv[:, :, 1], freqs, p["qn"], p["kn"], 1e-6)
        v = qkv[:, :, 2]
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            o = torch.nn.functional.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2),
                                                                 v.transpose(1, 2))
        o = o.transpose(1, 2).reshape(B * T, D)
        a = timed("w8a8", W.int8_linear, o, *p["out"])
        x = timed("glue", W.gated_residual, x, a.view(B, T, D), (mt[2], mi[2]), T_txt)
        q2, s2 = timed("norm_quant", W.modulated_norm_quant, x, (mt[4], mi[4]), T_txt, zero, 1e-6)
        up = timed("w8a8", W.gemm_dequant, q2, p["up"][0], s2, *p["up"][1:], torch.bfloat16)
        d = timed("w8a8", W.int8_linear, up, *p["down"], input_act="gelu_tanh")
        return timed("glue", W.gated_residual, x, d.view(B, T, D), (mt[5], mi[5]), T_txt)

    def step():
        x = x0.clone()
        for p in blks:
            x = block(x, p)
        return x

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    for v in ev.values():
        v.clear()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        out = step()
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / steps
    w8 = sum(a.elapsed_time(b) for a, b in ev["w8a8"]) / steps
    gl = sum(a.elapsed_time(b) for a, b in ev["glue"]) / steps
    nq = sum(a.elapsed_time(b) for a, b in ev["norm_quant"]) / steps
    ops = blocks * 2 * (B * T * D * (3 * D + D + FFN) + B * T * FFN * D + 2 * B * D * 6 * D)
    finite = bool(torch.isfinite(out).all())
    del blks
    return {"ms_per_step": round(ms, 2), "w8a8_ms": round(w8, 2), "w8a8_share": round(w8 / ms, 3),
            "w8a8_TOPS": round(ops / (w8 * 1e-3) / 1e12, 1), "glue_ms": round(gl, 2),
            "glue_share": round(gl / ms, 3), "norm_quant_ms": round(nq, 2), "norm_quant_share": round(nq / ms, 3),
            "blocks": blocks, "M": B * T, "steps": steps,
            "output_finite": finite,
            "rest": "attention (torch fused SDPA) and the head split / merge copies"}


def run_only(args, W, lib, dev, layers, step, quant, gemm, qbuf, x_ffn, outs):
    """One kernel in a loop (for rocprofv3 --pmc / --kernel-trace runs)."""
    n_iter = max(args.steps, 1)
    if args.only == "up_gemm":
        quant(x_ffn, qbuf[HID])
        for _ in range(n_iter):
            gemm(qbuf[HID], layers[2], outs["up"], True)
    elif args.only == "quant":
        for _ in range(n_iter):
            quant(x_ffn, qbuf[HID])
    elif args.only == "quant12288":
        x12 = torch.randn(M_TOK, FFN, device=dev).to(torch.bfloat16)
        q12 = torch.empty(M_TOK, FFN, dtype=torch.int8, device=dev)
        s12 = torch.empty(M_TOK, dtype=torch.float32, device=dev)
        for _ in range(n_iter):
            W._lib.check(lib.w8a8_quantize_rowwise(x12.data_ptr(), W._lib.BF16, q12.data_ptr(), s12.data_ptr(),
                                                   M_TOK, FFN, 0, torch.cuda.current_stream().cuda_stream))
    elif args.only == "gemv":
        # adaLN GEMV M=2 K=3072 N=18432 (one weight; the timed extra rotates 8)
        m, k, n = 2, HID, 6 * HID
        w, ws, b = make_linear(k, n, 40, dev)
        qg = torch.randint(-127, 128, (m, k), device=dev, dtype=torch.int8)
        xsg = torch.rand(m, device=dev) * 1e-2
        og = torch.empty(m, n, device=dev, dtype=torch.bfloat16)
        for _ in range(n_iter):
            W._lib.check(lib.w8a8_gemv_dequant(qg.data_ptr(), w.data_ptr(), xsg.data_ptr(), ws.data_ptr(), n,
                                               b.data_ptr(), og.data_ptr(), W._lib.BF16, m, n, k, 0,
                                               torch.cuda.current_stream().cuda_stream))
    elif args.only == "convrot_quant":
        s = torch.empty(M_TOK, dtype=torch.float32, device=dev)
        for _ in range(n_iter):
            W._lib.check(lib.w8a8_quantize_rowwise_convrot(x_ffn.data_ptr(), W._lib.BF16, qbuf[HID].data_ptr(),
                                                           s.data_ptr(), M_TOK, HID, 256, 0, None, 0,
                                                           torch.cuda.current_stream().cuda_stream))
    elif args.only == "step":
        for _ in range(n_iter):
            step()
    elif args.only == "rms_rope":
        # QK RMSNorm + RoPE on q / k views into a [2, 5856, 3, 24, 128] bf16 QKV output
        hb, ht, nh, hd = 2, M_TOK // 2, 24, HID // 24
        qkv = torch.randn(hb, ht, 3, nh, hd, device=dev).to(torch.bfloat16)
        qo = torch.empty(hb, ht, nh, hd, device=dev, dtype=torch.bfloat16)
        ko = torch.empty_like(qo)
        fr = torch.randn(ht, hd // 2, 2, 2, device=dev)
        sc = torch.ones(hd, device=dev, dtype=torch.bfloat16)
        for _ in range(n_iter):
            W._lib.check(lib.w8a8_rms_rope(qkv.data_ptr(), qkv[:, :, 1].data_ptr(), fr.data_ptr(), sc.data_ptr(),
                                           sc.data_ptr(), qo.data_ptr(), ko.data_ptr(), hb, ht, nh, hd, 3 * nh * hd,
                                           0, 1e-6, W._lib.BF16, torch.cuda.current_stream().cuda_stream))
    elif args.only == "copy":
        # counter calibration: a plain device copy of known size (1 GiB read,
        # 1 GiB written per launch) for scaling FETCH_SIZE / WRITE_SIZE
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(n_iter):
            dst.copy_(src)
    else:
        raise SystemExit(f"unknown --only {args.only}")
    torch.cuda.synchronize()
    print(f"[bench] ran {args.only} x{n_iter}", file=sys.stderr, flush=True)


if __name__ == "__main__":
    main()
