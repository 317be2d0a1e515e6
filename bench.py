"""Benchmark of the fused per-token layer kernels on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

A step is one launch of the headline kernel over the whole batch: the AdaLN chain (LayerNorm without affine, then x
* (1 + scale) + shift, GELU-tanh, out = res + gate * y) on X, res [16896 x 4096] bf16, token grid T16 x H24 x W44.
``value`` is its achieved HBM bandwidth: algorithmic bytes (X and res read once, out written once) divided by the
mean kernel time. Each kernel first runs untimed for 0.15 s (``--settle``; the clocks ramp up over the first
milliseconds of load), then W warm-up launches, then the K timed launches. The library context wraps PyTorch's
current stream (h3s_create), so the kernels run on that stream and the HIP events recorded on it (torch.cuda.Event)
bracket exactly the timed launches; inputs are already in HBM. The other fused kernels are timed the same way and
reported under ``kernels``; the int8 GEMM also as int8 TOPS. ``roofline.traffic`` is the headline kernel's HBM bytes
per launch from the rocprofv3 FETCH_SIZE / WRITE_SIZE runs summarized in profiles/hbm_traffic_pmc.md (each counter
scaled by what it reads for a 1 GiB device copy). ``cpu_baseline`` times the CPU oracle (the C restatement of the
reference arithmetic) on the same workload on this host. Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_GBS = 8000.0          # MI355X HBM3E
PEAK_I8_TOPS = 5000.0      # MI355X dense int8 matrix peak
PEAK_F16_TFLOPS = 2500.0   # MI355X dense fp16 / bf16 matrix peak

M2 = 16 * 24 * 44          # 16896 tokens (T16 x H24 x W44)
M4 = 47104
C = 4096


def bytes_cfg():
    """Algorithmic bytes per launch (minimum HBM traffic: every input read once, every output written once)."""
    return {
        "cfg1_rmsnorm_quant_2159": 2159 * C * 2 + 2159 * C + 2159 * 4,
        "cfg2_ln_mod_gelu_gate_16896": 3 * M2 * C * 2,
        "cfg3_qk_rmsnorm_rope3d_16896": 4 * M2 * 32 * 128 * 2 + M2 * 64 * 2 * 4,
        "cfg4_rmsnorm_wht128_quant_47104": M4 * C * 2 + M4 * C + M4 * 4,
        "cfg5a_rmsnorm_mod_quant_47104": M4 * C * 2 + M4 * C + M4 * 4,
        "cfg5b_int8_gemm_silu_47104x16384": M4 * C + 16384 * C + M4 * 4 + 16384 * 4 + M4 * 16384 * 2,
        "mlp_swiglu_quant_g256_47104x8192": M4 * 16384 * 2 + M4 * 8192 + M4 * 4,
        # the other token count of the measured pair (16.8k and 47k tokens x 4096) for configs 2-5a
        "cfg2_ln_mod_gelu_gate_47104": 3 * M4 * C * 2,
        "cfg3_qk_rmsnorm_rope3d_47104": 4 * M4 * 32 * 128 * 2 + M4 * 64 * 2 * 4,
        "cfg4_rmsnorm_wht128_quant_16896": M2 * C * 2 + M2 * C + M2 * 4,
        "cfg5a_rmsnorm_mod_quant_16896": M2 * C * 2 + M2 * C + M2 * 4,
        "attn_sage_16896x32x128": 4 * M2 * 4096 * 2,     # q, k, v read, out written (the products are the bound)
        "attn_sage_47104x32x128": 4 * M4 * 4096 * 2,
    }


def measured_traffic(key):
    """HBM bytes per launch of kernel `key` from the committed counter summary, scaled by the copy calibration."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic_pmc.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic:") and line.split()[1] == key:
                    kv = dict(t.split("=") for t in line.split()[2:])
                    cal_f = float(kv["copy_kib"]) / float(kv["copy_fetch_kib"])
                    cal_w = float(kv["copy_kib"]) / float(kv["copy_write_kib"])
                    return int(round((float(kv["fetch_kib"]) * cal_f + float(kv["write_kib"]) * cal_w) * 1024))
    except (OSError, KeyError, ValueError):
        return None
    return None


def rope_table(T, Hh, Ww, dims=(32, 48, 48), theta=10000.0):
    """(cos, sin) per token and rotated pair [M, 64, 2], float32: positions from the grid, angle = pos * theta^(-2i/d)
    per axis in float32, the axes one after the other (engine/h3-core/src/dit.rs:190-203)."""
    import numpy as np

    t, h, w = np.meshgrid(np.arange(T), np.arange(Hh), np.arange(Ww), indexing="ij")
    pos = np.stack([t.ravel(), h.ravel(), w.ravel()], -1).astype(np.float32)
    cols = []
    for a, d in enumerate(dims):
        inv = (np.float32(1.0) / np.power(np.float32(theta), np.arange(0, d, 2, dtype=np.float32) / np.float32(d))).astype(np.float32)
        cols.append(pos[:, a:a + 1] * inv[None, :])
    ang = np.concatenate(cols, 1).astype(np.float32)
    return np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--settle", type=float, default=0.15, help="seconds each kernel runs untimed before its warm-up")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default="", help="comma list of kernel keys to time (default all)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also time a plain device copy of 1 GiB (the attainable HBM rate; the known-size kernel that "
                         "scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: one GPU only; --gpus {args.gpus} is not supported (the per-token kernels would shard by "
              "contiguous token rows with no exchange step, so one GPU's share is the measured workload)", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from sycl_minimax_h3_amd import Device, DType, Tensor, ops
    import sycl_minimax_h3_amd.api as A

    torch.manual_seed(0)
    dev_t = torch.device("cuda:0")
    dev = Device.from_torch()
    T = lambda t, dt=None: Tensor.from_torch(t, dt, dev)   # noqa: E731
    B = bytes_cfg()
    only = set(filter(None, args.only.split(",")))

    def bf16(*shape, scale=1.0):
        return (torch.randn(*shape, device=dev_t) * scale).to(torch.bfloat16)

    def timed(fn, steps, warmup, settle_s=args.settle):
        # The device's clocks ramp up over the first ~10 ms of sustained load: before the W warm-up launches, keep
        # launching (untimed) until settle_s seconds of this kernel have run, so the timed launches see the sustained
        # state a busy serving loop runs in.
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < settle_s:
            for _ in range(10):
                fn()
            torch.cuda.synchronize()
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps   # ms per launch

    kernels = {}

    # ---- config 2 (headline): LN (no affine) -> * (1 + scale) + shift -> GELU-tanh -> res + gate * y ----
    x2, r2, o2 = bf16(M2, C), bf16(M2, C), torch.empty(M2, C, dtype=torch.bfloat16, device=dev_t)
    tab = [bf16(1, C, scale=0.5) for _ in range(3)]
    tb2 = ops.Tables(scale=T(tab[0]), shift=T(tab[1]), gate=T(tab[2]))
    X2, R2, O2 = T(x2), T(r2), T(o2)
    f2 = lambda: ops.norm_mod_act_gate(X2, A.NORM_LAYER, None, None, 1e-5, tb2, A.ACT_GELU_TANH, R2, O2)  # noqa: E731
    ms2 = timed(f2, args.steps, args.warmup)
    kernels["cfg2_ln_mod_gelu_gate_16896"] = ms2

    def run(key, fn, steps=20):
        if only and key not in only:
            return
        kernels[key] = timed(fn, steps, 3)

    # ---- config 1: RMSNorm (eps 1e-6) + per-token int8 quant, [2159 x 4096] ----
    x1 = bf16(2159, C)
    g1 = (1 + 0.1 * torch.randn(C, device=dev_t)).float()
    q1, s1 = torch.empty(2159, C, dtype=torch.int8, device=dev_t), torch.empty(2159, device=dev_t)
    X1, G1, Q1, S1 = T(x1), T(g1), T(q1), T(s1)
    run("cfg1_rmsnorm_quant_2159", lambda: ops.norm_quant(X1, G1, 1e-6, None, Q1, S1), 200)

    # ---- config 3: qk-RMSNorm + 3D RoPE in place, q, k [16896 x 32 x 128], split 32/48/48 ----
    q3, k3 = bf16(M2, 32 * 128), bf16(M2, 32 * 128)
    wq, wk = (1 + 0.1 * torch.randn(128, device=dev_t)).float(), (1 + 0.1 * torch.randn(128, device=dev_t)).float()
    cs = torch.from_numpy(rope_table(16, 24, 44)).to(dev_t)
    Q3, K3, WQ, WK, CS = T(q3), T(k3), T(wq), T(wk), T(cs)
    run("cfg3_qk_rmsnorm_rope3d_16896", lambda: ops.qk_rms_rope(ops.Rows(Q3, 0, 4096, M2, 32, 128), ops.Rows(K3, 0, 4096, M2, 32, 128),
                                                                 WQ, WK, 1e-5, CS, 128))

    # ---- config 4: RMSNorm -> Sylvester WHT-128 -> int8 quant, [47104 x 4096], 1% of channels x20 ----
    ch = torch.randperm(C, generator=torch.Generator().manual_seed(4))[:41].to(dev_t)
    x4 = torch.randn(M4, C, device=dev_t)
    x4[:, ch] *= 20
    x4 = x4.to(torch.bfloat16)
    q4, s4 = torch.empty(M4, C, dtype=torch.int8, device=dev_t), torch.empty(M4, device=dev_t)
    X4, Q4, S4 = T(x4), T(q4), T(s4)
    run("cfg4_rmsnorm_wht128_quant_47104", lambda: ops.norm_quant(X4, G1, 1e-6, None, Q4, S4, rot=A.ROT_SYLVESTER, group=128))

    # ---- config 5a: RMSNorm + modulate + int8 quant, [47104 x 4096]; 5b: int8 GEMM + dequant + SiLU ----
    x5 = bf16(M4, C)
    sc5, sh5 = bf16(1, C, scale=0.5), bf16(1, C, scale=0.5)
    tb5 = ops.Tables(scale=T(sc5), shift=T(sh5))
    X5 = T(x5)
    run("cfg5a_rmsnorm_mod_quant_47104", lambda: ops.norm_quant(X5, G1, 1e-6, tb5, Q4, S4))
    w5 = torch.randint(-127, 128, (16384, C), dtype=torch.int8, device=dev_t)
    ws5 = (0.005 + 0.015 * torch.rand(16384, device=dev_t)).float()
    out5 = bf16(M4, 16384)
    layer = ops.Int8Linear(T(w5), T(ws5))
    O5 = T(out5)
    run("cfg5b_int8_gemm_silu_47104x16384", lambda: ops.int8_gemm_dequant(Q4, S4, layer, A.ACT_SILU, O5), 5)

    # ---- the MLP's middle: swiglu of fc1's [gate | up] output [47104 x 2*8192] -> fc2's quantizer (regular g 256) ----
    q6, s6 = torch.empty(M4, 8192, dtype=torch.int8, device=dev_t), torch.empty(M4, device=dev_t)
    X6, Q6, S6 = O5, T(q6), T(s6)    # the GEMM's output rows are [gate | up] halves of 8192
    run("mlp_swiglu_quant_g256_47104x8192", lambda: ops.swiglu_quant(X6, Q6, S6, rot=A.ROT_REGULAR, group=256))

    # ---- configs 2-5a at the other token count: 47104 tokens (grid T46 x H32 x W32) for 2 and 3, 16896 for 4 and 5a ----
    x2b, r2b, o2b = bf16(M4, C), bf16(M4, C), torch.empty(M4, C, dtype=torch.bfloat16, device=dev_t)
    X2b, R2b, O2b = T(x2b), T(r2b), T(o2b)
    run("cfg2_ln_mod_gelu_gate_47104", lambda: ops.norm_mod_act_gate(X2b, A.NORM_LAYER, None, None, 1e-5, tb2, A.ACT_GELU_TANH, R2b, O2b))
    del x2b, r2b, o2b, X2b, R2b, O2b
    q3b, k3b = bf16(M4, 32 * 128), bf16(M4, 32 * 128)
    cs3b = torch.from_numpy(rope_table(46, 32, 32)).to(dev_t)
    Q3b, K3b, CS3b = T(q3b), T(k3b), T(cs3b)
    run("cfg3_qk_rmsnorm_rope3d_47104", lambda: ops.qk_rms_rope(ops.Rows(Q3b, 0, 4096, M4, 32, 128), ops.Rows(K3b, 0, 4096, M4, 32, 128),
                                                                 WQ, WK, 1e-5, CS3b, 128))
    del q3b, k3b, cs3b, Q3b, K3b, CS3b
    X4s, Q4s, S4s, X5s = T(x4[:M2]), T(q4[:M2]), T(s4[:M2]), T(x5[:M2])
    run("cfg4_rmsnorm_wht128_quant_16896", lambda: ops.norm_quant(X4s, G1, 1e-6, None, Q4s, S4s, rot=A.ROT_SYLVESTER, group=128))
    run("cfg5a_rmsnorm_mod_quant_16896", lambda: ops.norm_quant(X5s, G1, 1e-6, tb5, Q4s, S4s))

    # ---- attention of the 16896-token grid, 32 heads of 128 (the int8 form: S >= 8192) ----
    qkv7 = bf16(M2, 3 * 4096)
    o7 = torch.empty(M2, 4096, dtype=torch.bfloat16, device=dev_t)
    QKV7, O7 = T(qkv7), T(o7)
    rows7 = [ops.Rows(QKV7, i * 4096, 3 * 4096, M2, 32, 128) for i in range(3)]
    run("attn_sage_16896x32x128", lambda: ops.attention(*rows7, O7), 10)
    del qkv7, o7, QKV7, O7, rows7
    # the same at 47104 tokens (the 47k configurations' sequence)
    qkv8 = bf16(M4, 3 * 4096)
    o8 = torch.empty(M4, 4096, dtype=torch.bfloat16, device=dev_t)
    QKV8, O8 = T(qkv8), T(o8)
    rows8 = [ops.Rows(QKV8, i * 4096, 3 * 4096, M4, 32, 128) for i in range(3)]
    run("attn_sage_47104x32x128", lambda: ops.attention(*rows8, O8), 3)
    del qkv8, o8, QKV8, O8, rows8

    copy = None
    if args.copy_probe:
        src = torch.empty(1 << 29, dtype=torch.bfloat16, device=dev_t).fill_(1.0)
        dst = torch.empty_like(src)
        ms_c = timed(lambda: dst.copy_(src), 20, 3)
        copy = {"bytes": 2 * src.numel() * 2, "ms": round(ms_c, 4), "GB/s": round(2 * src.numel() * 2 / (ms_c * 1e-3) / 1e9, 1)}
        del src, dst

    per = {}
    for k, ms in kernels.items():
        gbs = B[k] / (ms * 1e-3) / 1e9
        e = {"ms": round(ms, 5), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_GBS, 4), "bytes": B[k]}
        if k.startswith("cfg5b"):
            tops = 2 * M4 * C * 16384 / (ms * 1e-3) / 1e12
            e.update({"TOPS_i8": round(tops, 1), "frac_i8_peak": round(tops / PEAK_I8_TOPS, 4)})
        if k.startswith("attn"):
            # q k^T on the i8 cores (5 POPS) and P v on the f16 cores (2.5 PFLOP/s): the time both take at peak
            S_ = M2 if "16896" in k else M4
            half_ops = 2.0 * S_ * S_ * 4096
            t_peak = half_ops / (PEAK_I8_TOPS * 1e12) + half_ops / (PEAK_F16_TFLOPS * 1e12)
            e.update({"TOPS": round(2 * half_ops / (ms * 1e-3) / 1e12, 1), "frac_mfma_peak": round(t_peak / (ms * 1e-3), 4)})
        per[k] = e

    value = B["cfg2_ln_mod_gelu_gate_16896"] / (ms2 * 1e-3) / 1e9
    line = {
        "metric": "achieved HBM GB/s (% of 8 TB/s) per fused kernel at 16.8k/47k tokens x 4096",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms2, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (torch.randn on the device; shift/scale/gate ~N(0,0.5))",
        "config": {"workload": "AdaLN chain: LayerNorm(no affine) -> x*(1+scale)+shift -> GELU-tanh -> res + gate*y, "
                               "X,res [16896 x 4096] bf16 (grid T16xH24xW44)", "tokens": M2, "hidden": C},
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / PEAK_GBS, 4), "traffic": measured_traffic("cfg2_ln_mod_gelu_gate_16896")},
        "kernels": per,
        "device": dev.name(),
    }
    if copy:
        line["copy_probe"] = copy
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(x2, r2, tab, {"x1": x1, "g1": g1, "q3": q3, "k3": k3, "wq": wq, "wk": wk,
                                                          "cs": cs, "x4": x4, "x5": x5, "sc5": sc5, "sh5": sh5,
                                                          "q4": q4, "s4": s4, "w5": w5, "ws5": ws5})
    print(json.dumps(line), flush=True)
    return 0


def cpu_baseline(x2, r2, tab, t):
    """The CPU oracle (oracle/h3oracle.c, C restatement of the reference arithmetic, row-parallel with contiguous row
    chunks as engine/h3-core/src/reference.rs:43-80) on this host: the headline workload, and under `kernels` the other
    configurations on their full inputs (the GEMM on its first 1024 rows, scaled linearly), each the median of a few
    runs (about 10 s in all for the headline, a few runs for the others)."""
    import numpy as np
    import torch

    from oracle import oracle as o

    threads = min(16, os.cpu_count() or 1)
    o.set_threads(threads)
    u16 = lambda a: a.view(torch.int16).cpu().numpy().view(np.uint16).ravel()   # noqa: E731
    f32 = lambda a: a.float().cpu().numpy().ravel()                              # noqa: E731

    def median_time(fn, budget, least=3, most=50):
        fn()
        times = []
        t_end = time.perf_counter() + budget
        while len(times) < least or (time.perf_counter() < t_end and len(times) < most):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return float(np.median(times)), len(times)

    x, r = u16(x2), u16(r2)
    tb = [u16(a) for a in tab]
    med, n = median_time(lambda: o.norm_mod_act_gate(x, o.BF16, M2, C, o.NORM_LAYER, None, None, 1e-5, None, tb[0], tb[1],
                                                     tb[2], o.BF16, o.ACT_GELU_TANH, r, o.BF16, o.BF16), 10.0)
    B = bytes_cfg()
    gbs = B["cfg2_ln_mod_gelu_gate_16896"] / med / 1e9
    cpu = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            cpu = next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except Exception:
        pass
    out = {"value": round(gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
           "sample": f"the full 16896 x 4096 workload, median of {n} runs ({med * 1e3:.1f} ms each) on {cpu}"}

    # the other configurations, on the same tensors the GPU ran
    per = {}
    x1, g1 = u16(t["x1"]), f32(t["g1"])
    m, _ = median_time(lambda: o.norm_quant(x1, o.BF16, 2159, C, g1, 1e-6), 2.0)
    per["cfg1_rmsnorm_quant_2159"] = m
    q3, k3, wq, wk, cs = u16(t["q3"]), u16(t["k3"]), f32(t["wq"]), f32(t["wk"]), f32(t["cs"])
    m, _ = median_time(lambda: (o.rms_rope(q3, o.BF16, M2, 32, 128, 4096, wq, 1e-5, cs, 128),
                                o.rms_rope(k3, o.BF16, M2, 32, 128, 4096, wk, 1e-5, cs, 128)), 2.0)
    per["cfg3_qk_rmsnorm_rope3d_16896"] = m
    x4 = u16(t["x4"])
    m, _ = median_time(lambda: o.norm_quant(x4, o.BF16, M4, C, g1, 1e-6, rot=o.ROT_SYLVESTER, group=128), 2.0)
    per["cfg4_rmsnorm_wht128_quant_47104"] = m
    x5, sc5, sh5 = u16(t["x5"]), u16(t["sc5"]), u16(t["sh5"])
    m, _ = median_time(lambda: o.norm_quant(x5, o.BF16, M4, C, g1, 1e-6, None, sc5, sh5, o.BF16), 2.0)
    per["cfg5a_rmsnorm_mod_quant_47104"] = m
    rows = 1024
    q4 = t["q4"][:rows].cpu().numpy().ravel()
    s4 = t["s4"][:rows].cpu().numpy().ravel()
    w5, ws5 = t["w5"].cpu().numpy().ravel(), f32(t["ws5"])
    m, _ = median_time(lambda: o.gemm_dequant(q4, s4, rows, C, w5, 16384, ws5, act=o.ACT_SILU), 2.0, least=2)
    per["cfg5b_int8_gemm_silu_47104x16384"] = m * M4 / rows
    kernels = {}
    for k, sec in per.items():
        e = {"ms": round(sec * 1e3, 3), "GB/s": round(B[k] / sec / 1e9, 2)}
        if k.startswith("cfg5b"):
            e["TOPS_i8"] = round(2 * M4 * C * 16384 / sec / 1e12, 3)
            e["sample"] = f"the first {rows} of {M4} rows, time scaled by {M4 / rows:.1f}"
        kernels[k] = e
    out["kernels"] = kernels
    return out


if __name__ == "__main__":
    sys.exit(main())
