"""Benchmark of the fused per-token layer kernels on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only k1,k2] [--mark] [--copy-probe]
    python bench.py --summarize-trace TRACE.csv --bench-json BENCH.json           (a profiles/ table, see below)
    python bench.py --summarize-pmc COUNTERS.csv [COUNTERS2.csv] --bench-json BENCH.json

A step is one launch of the headline kernel over the whole batch: the AdaLN chain (LayerNorm without affine, then
x * (1 + scale) + shift, GELU-tanh, out = res + gate * y) on X, res [16896 x 4096] bf16, token grid T16 x H24 x W44.
``value`` is its achieved HBM bandwidth: algorithmic bytes (X and res read once, out written once) divided by the
median launch time (the timed launches run back to back in up to 5 equal windows between HIP events: the median of the
windows' times per launch; the mean over all of them is reported beside it).

Cache-cold timing: MI355X's 256 MB Infinity Cache would hold part of a 415 MB working set launched back to back on
the same buffers. Every workload of less than 1 GiB per launch is therefore timed over a ring of independent buffer
sets whose footprint is at least 1 GiB (3 sets for the headline), one set per launch in turn: a launch never finds
its inputs in the cache. The headline's back-to-back figure on one set is reported beside it.

Each kernel first runs untimed for 0.15 s (``--settle``; the clocks ramp up over the first milliseconds of load), then
W warm-up launches, then the K timed launches, bracketed by HIP events on the stream the kernels run on (the library
context wraps PyTorch's current stream, h3s_create). Inputs are already in HBM. The other fused kernels are timed the
same way and reported under ``kernels``; the int8 GEMM also as int8 TOPS and attention against the mixed int8 / fp16
matrix peak. The compute-bound ones (the int8 GEMM, attention) are timed after the HBM-bound ones, whose clock a third
of a second of the GEMM would lower. ``roofline.traffic`` is the headline kernel's HBM bytes per launch from the
rocprofv3 FETCH_SIZE / WRITE_SIZE runs summarized in profiles/hbm_traffic_pmc.md (each counter scaled by what it reads
for a 1 GiB device copy). ``cpu_baseline`` times the CPU oracle (the C restatement of the reference arithmetic) on the
same workload on this host.

``--copy-probe`` also times two plain device copies: 1 GiB (the attainable streaming rate, and the known-size kernel
that scales the byte counters) and config 1's 26.5 MB (the floor a launch of that size reaches from a cold cache).

``--mark`` launches a one-cycle spin kernel right before and right after each timed region (outside its HIP
events), so a rocprofv3 trace of the run can be cut into exactly the timed dispatches of each workload; the bench
line then lists the marked workloads in order. ``--summarize-trace`` and ``--summarize-pmc`` turn such a trace
(kernel trace or counter collection, rocprofv3 ``-f csv``) and the bench line of the same run into the tables
committed under profiles/. Prints one JSON line.
"""
from __future__ import annotations

import argparse
import collections
import csv
import fnmatch
import json
import math
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_GBS = 8000.0          # MI355X HBM3E
PEAK_I8_TOPS = 5000.0      # MI355X dense int8 matrix peak
PEAK_F16_TFLOPS = 2500.0   # MI355X dense fp16 / bf16 matrix peak
RING_BYTES = 1 << 30       # the least footprint of a ring of buffer sets (4x the Infinity Cache)
MARKER = "spin_kernel"     # the kernel torch.cuda._sleep launches: the --mark boundaries

M2 = 16 * 24 * 44          # 16896 tokens (T16 x H24 x W44)
M4 = 47104
C = 4096
HEADLINE = "cfg2_ln_mod_gelu_gate_16896"
CFG1_COPY_ELEMS = (2159 * C * 2 + 2159 * C + 2159 * 4) // 4      # bf16 elements: read + write = config 1's bytes


def bytes_cfg():
    """Algorithmic bytes per launch (minimum HBM traffic: every input read once, every output written once)."""
    return {
        HEADLINE: 3 * M2 * C * 2,
        HEADLINE + "_same_buffers": 3 * M2 * C * 2,
        "cfg1_rmsnorm_quant_2159": 2159 * C * 2 + 2159 * C + 2159 * 4,
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
        "attn_f16_4096x32x128": 4 * 4096 * 4096 * 2,     # the 16-bit form (below 8192 tokens)
        **dit_bytes(M2), **dit_bytes(M4), **float_linear_bytes(M2), **lora_bytes(M4),
        "copy_probe_1GiB": 2 << 30,
        # a plain copy moving config 1's bytes (half read, half written): the floor a launch of that size reaches
        "copy_probe_cfg1_bytes": 2 * CFG1_COPY_ELEMS * 2,
        # torch's own elementwise kernels with the traffic of the fused kernels, the rate this device streams such a
        # shape at: out = x + res (the AdaLN chain's two reads and one write), the two halves of each row of x added
        # into a row half as long (the quantizers' 2 bytes read and 1 written a feature; torch's bfloat16 -> int8
        # cast of the same bytes runs at 17 % of 8 TB/s), q of the qkv rows scaled in place (the DiT's rope)
        **{f"probe_add_bf16_{M}x{C}": 3 * M * C * 2 for M in (M2, M4)},
        **{f"probe_halfadd_bf16_{M}x{C}": M * C * 3 for M in (M2, M4)},
        **{f"probe_inplace_bf16_{M}x7168_of_21504": 2 * M * 7168 * 2 for M in (M2, M4)},
    }


# The DiT block of the denoiser as the unchanged engine runs it (engine/h3-core/src/dit.rs:329-369): hidden 5376, 56
# heads of 128 (q, k, v side by side in rows of 3 x 7168), an MLP of 5376 -> 2 x 14336 -> 5376 (docs/BASELINE.md:13),
# rot_dim = 6 x 21 frequencies = 126 (dit.rs:71), float32 modulation tables [2, 5376] with the first 5 % of the
# tokens on table row 1 (engine/h3d/src/jobs.rs:213), every activation bfloat16 (jobs.rs:217).
DH, DHEADS, DHD, DFF, DROT = 5376, 56, 128, 14336, 126
DQKV = 3 * DHEADS * DHD
# the block's int8 linears: (name, K, N), dit.rs:341, 352, 359, 364
DIT_LINEARS = (("qkv", DH, DQKV), ("out", DHEADS * DHD, DH), ("fc1", DH, 2 * DFF), ("fc2", DFF, DH))
# the block's stages under the labels of the reference's harness (engine/h3d/src/jobs.rs:269-279), each the sum of
# the workloads that run it, and the engine's published times per block (docs/PORT-PLAN.md:62-70, on its GPU)
DIT_STAGES = (
    ("norm + scale/shift", ("dit_rms_norm_mod", "dit_rms_norm_mod")),
    ("linear: q, k, v", ("dit_int8_linear_qkv",)),
    ("per-head norm + rotation (q, k)", ("dit_rms_rope_q_rot126", "dit_rms_rope_k_rot126")),
    ("attention", ("dit_attention",)),
    ("linear: attention out", ("dit_int8_linear_out",)),
    ("gated add", ("dit_gate_add", "dit_gate_add")),
    ("linear: MLP in", ("dit_int8_linear_fc1",)),
    ("gated activation + linear: MLP out", ("dit_swiglu", "dit_int8_linear_fc2")),
)
DIT_PUBLISHED_MS = {"16.5k tokens": {"the four int8 linears (+ gated activation)": 67, "per-head norm + rotation": 6.2,
                                     "norms, scale/shift, gated adds": 10.5, "attention": 96, "the block": 177},
                    "47k tokens": {"the four int8 linears (+ gated activation)": 194, "per-head norm + rotation": 20.8,
                                   "norms, scale/shift, gated adds": 28.1, "attention": 759, "the block": 998}}


def dit_bytes(M: int) -> dict:
    """Algorithmic bytes per launch of the DiT block's workloads at M tokens."""
    cs126, cs96 = M * DROT // 2 * 2 * 4, M * 48 * 2 * 4
    out = {
        f"dit_rms_norm_mod_{M}": 2 * M * DH * 2 + M * 4,                  # x read, h written, the row table
        f"dit_rms_rope_q_rot126_{M}": 2 * M * DHEADS * DHD * 2 + cs126,   # q read and written in place, cos/sin
        f"dit_rms_rope_k_rot126_{M}": 2 * M * DHEADS * DHD * 2 + cs126,
        f"dit_rms_rope_q_rot96_{M}": 2 * M * DHEADS * DHD * 2 + cs96,
        f"dit_qk_rms_rope_rot126_{M}": 4 * M * DHEADS * DHD * 2 + cs126,  # the fused pair: cos/sin read once
        f"dit_gate_add_{M}": 3 * M * DH * 2 + M * 4,                      # x read and written, the projection read
        f"dit_swiglu_{M}": M * 2 * DFF * 2 + M * DFF * 2,
        f"dit_norm_quant_g256_{M}": M * DH * 2 + M * DH + M * 4 + M * 4,  # x read, codes and scales, the row table
        f"dit_swiglu_quant_g256_{M}": M * 2 * DFF * 2 + M * DFF + M * 4,
        f"dit_attention_{M}": 4 * M * DHEADS * DHD * 2,
    }
    for name, K, N in DIT_LINEARS:
        out[f"dit_quantize_g256_{name}_{M}"] = M * K * 2 + M * K + M * 4     # the int8 linear's first pass
        out[f"dit_int8_linear_{name}_{M}"] = M * K * 2 + N * K + N * 4 + M * N * 2
    return out


# The float linear (h3s_linear / h3s_linear_acc) at the DiT's hidden width, bfloat16 activations: a linear of the
# width (with a bias) and a LoRA's two products at rank 64 (engine/h3-core/src/ops.rs:146-160: tmp = A x, then
# out += B tmp); and torch's bfloat16 matmul of the square shape (the vendor library's rate, no bias)
LORA_RANK = 64
FLOAT_LINEARS = (("linear_bf16", DH, DH, True, False), ("lora_a_bf16", DH, LORA_RANK, False, False),
                 ("lora_b_acc_bf16", LORA_RANK, DH, False, True))


def float_linear_bytes(M: int) -> dict:
    out = {}
    for name, K, N, bias, acc in FLOAT_LINEARS:
        out[f"{name}_{M}x{K}x{N}"] = M * K * 2 + N * K * 2 + (N * 4 if bias else 0) + M * N * 2 * (2 if acc else 1)
    out[f"probe_matmul_bf16_{M}x{DH}x{DH}"] = M * DH * 2 + DH * DH * 2 + M * DH * 2
    return out


def lora_bytes(M: int) -> dict:
    """the LoRA factors alone at another token count"""
    return {k: v for k, v in float_linear_bytes(M).items() if k.startswith("lora_")}


def ring_size(nbytes: int) -> int:
    """Buffer sets of a ring whose footprint is at least RING_BYTES (one set when a launch moves that much)."""
    return max(1, min(64, -(-RING_BYTES // nbytes)))


def measured_traffic(key):
    """HBM bytes per launch of workload `key` from the committed counter summary, scaled by the copy calibration."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic_pmc.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic:") and line.split()[1] == key:
                    kv = dict(t.split("=") for t in line.split()[2:])
                    return int(kv["bytes"])
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


def cpu_share() -> dict:
    """This host's CPUs as the process sees them: nproc, the affinity mask and the cgroup CPU quota (if any)."""
    out = {"nproc": os.cpu_count() or 1}
    try:
        out["affinity"] = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        out["affinity"] = out["nproc"]
    quota = None
    try:
        q, p = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if q != "max":
            quota = int(q) / int(p)
    except (OSError, ValueError):
        pass
    out["cgroup_quota"] = quota
    try:
        with open("/proc/cpuinfo") as f:
            out["model"] = next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except Exception:
        out["model"] = "unknown"
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--settle", type=float, default=0.15, help="seconds each kernel runs untimed before its warm-up")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default="", help="comma list of workload keys or shell-style patterns to time (default all)")
    ap.add_argument("--mark", action="store_true", help="bracket each timed region with a spin-kernel marker")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also time plain device copies of 1 GiB (the attainable HBM rate; the known-size kernel that "
                         "scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters) and of config 1's 26.5 MB")
    ap.add_argument("--summarize-trace", default="", help="a rocprofv3 kernel trace csv of a --mark run: print a table")
    ap.add_argument("--summarize-pmc", nargs="+", default=[], help="rocprofv3 counter csv(s) of --mark runs")
    ap.add_argument("--bench-json", default="", help="the bench line of the profiled run (for --summarize-*)")
    args = ap.parse_args()
    if args.summarize_trace:
        print(summarize_trace(args.summarize_trace, args.bench_json))
        return 0
    if args.summarize_pmc:
        print(summarize_pmc(args.summarize_pmc, args.bench_json))
        return 0
    if args.gpus != 1:
        print(f"bench.py: one GPU only; --gpus {args.gpus} is not supported (the per-token kernels would shard by "
              "contiguous token rows with no exchange step, so one GPU's share is the measured workload)", file=sys.stderr)
        return 2

    import numpy as np  # noqa: F401
    import torch

    from sycl_minimax_h3_amd import Device, Tensor, ops
    import sycl_minimax_h3_amd.api as A

    torch.manual_seed(0)
    dev_t = torch.device("cuda:0")
    dev = Device.from_torch()
    T = lambda t, dt=None: Tensor.from_torch(t, dt, dev)   # noqa: E731
    B = bytes_cfg()
    only = set(filter(None, args.only.split(",")))

    def skip(key):
        """not among --only's keys (shell-style patterns: dit_*rope* takes every key that matches)"""
        return bool(only) and not any(fnmatch.fnmatchcase(key, k) for k in only)
    marked, steps_of = [], {}

    def bf16(*shape, scale=1.0):
        return (torch.randn(*shape, device=dev_t) * scale).to(torch.bfloat16)

    def timed(key, fn, steps, warmup, settle_s=args.settle):
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
        steps_of[key] = steps
        if args.mark:
            torch.cuda._sleep(1)
            marked.append(key)
        # The launches back to back in up to 5 windows of equal length, an event at each window's edge: the median of
        # the windows' times per launch, and the mean over all of them. (An event between every two launches puts its
        # own gap, about 3 us, into every launch's time.)
        nw = max(1, min(5, steps // 4))
        edges = [round(i * steps / nw) for i in range(nw + 1)]
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(nw + 1)]
        ev[0].record()
        for w in range(nw):
            for _ in range(edges[w + 1] - edges[w]):
                fn()
            ev[w + 1].record()
        if args.mark:
            torch.cuda._sleep(1)
        torch.cuda.synchronize()
        each = sorted(ev[w].elapsed_time(ev[w + 1]) / (edges[w + 1] - edges[w]) for w in range(nw))
        means[key] = ev[0].elapsed_time(ev[nw]) / steps
        return each[nw // 2] if nw % 2 else 0.5 * (each[nw // 2 - 1] + each[nw // 2])   # median ms a launch

    def cycle(fns):
        """one launch of the next buffer set of a ring"""
        state = [0]

        def f():
            fns[state[0] % len(fns)]()
            state[0] += 1
        return f

    kernels, rings, means = {}, {}, {}

    def run(key, make, steps=20, warmup=3, ring=None):
        """times workload `key`: make() builds one buffer set and returns its launch; a ring of them when small
        (ring: a fixed count instead)"""
        if skip(key):
            return
        n = ring or ring_size(B[key])
        fns = [make() for _ in range(n)]
        kernels[key] = timed(key, cycle(fns), steps, warmup)
        rings[key] = n
        del fns
        torch.cuda.empty_cache()

    # ---- config 2 (headline): LN (no affine) -> * (1 + scale) + shift -> GELU-tanh -> res + gate * y ----
    tab = [bf16(1, C, scale=0.5) for _ in range(3)]
    tb2 = ops.Tables(scale=T(tab[0]), shift=T(tab[1]), gate=T(tab[2]))
    first = {}

    def make2():
        x, r, o = bf16(M2, C), bf16(M2, C), torch.empty(M2, C, dtype=torch.bfloat16, device=dev_t)
        first.setdefault("x2", x)
        first.setdefault("r2", r)
        X, R, O = T(x), T(r), T(o)
        return lambda: ops.norm_mod_act_gate(X, A.NORM_LAYER, None, None, 1e-5, tb2, A.ACT_GELU_TANH, R, O)

    n2 = ring_size(B[HEADLINE])
    ring2 = [make2() for _ in range(n2)]
    ms2 = timed(HEADLINE, cycle(ring2), args.steps, args.warmup)
    kernels[HEADLINE], rings[HEADLINE] = ms2, n2
    # the same launches back to back on one buffer set: part of the 415 MB stays in the Infinity Cache
    if not skip(HEADLINE + "_same_buffers"):
        kernels[HEADLINE + "_same_buffers"] = timed(HEADLINE + "_same_buffers", ring2[0], args.steps, args.warmup)
        rings[HEADLINE + "_same_buffers"] = 1
    del ring2
    x2, r2 = first["x2"], first["r2"]

    # ---- config 1: RMSNorm (eps 1e-6) + per-token int8 quant, [2159 x 4096] ----
    g1 = (1 + 0.1 * torch.randn(C, device=dev_t)).float()
    G1 = T(g1)

    def make1():
        x = bf16(2159, C)
        first.setdefault("x1", x)
        X, Q, S = T(x), T(torch.empty(2159, C, dtype=torch.int8, device=dev_t)), T(torch.empty(2159, device=dev_t))
        return lambda: ops.norm_quant(X, G1, 1e-6, None, Q, S)
    run("cfg1_rmsnorm_quant_2159", make1, 200)
    if "x1" not in first:
        first["x1"] = bf16(2159, C)

    # ---- config 3: qk-RMSNorm + 3D RoPE in place, q, k [16896 x 32 x 128], split 32/48/48 ----
    wq, wk = (1 + 0.1 * torch.randn(128, device=dev_t)).float(), (1 + 0.1 * torch.randn(128, device=dev_t)).float()
    WQ, WK = T(wq), T(wk)
    cs = torch.from_numpy(rope_table(16, 24, 44)).to(dev_t)
    CS = T(cs)

    def make3(M, csT):
        def make():
            q, k = bf16(M, 32 * 128), bf16(M, 32 * 128)
            first.setdefault(f"q3_{M}", q)
            first.setdefault(f"k3_{M}", k)
            Qr, Kr = ops.Rows(T(q), 0, 4096, M, 32, 128), ops.Rows(T(k), 0, 4096, M, 32, 128)
            return lambda: ops.qk_rms_rope(Qr, Kr, WQ, WK, 1e-5, csT, 128)
        return make
    run("cfg3_qk_rmsnorm_rope3d_16896", make3(M2, CS))

    # ---- config 4: RMSNorm -> Sylvester WHT-128 -> int8 quant, 1% of channels x20 ----
    ch = torch.randperm(C, generator=torch.Generator().manual_seed(4))[:41].to(dev_t)

    def make4(M):
        def make():
            x = torch.randn(M, C, device=dev_t)
            x[:, ch] *= 20
            x = x.to(torch.bfloat16)
            first.setdefault(f"x4_{M}", x)
            X, Q, S = T(x), T(torch.empty(M, C, dtype=torch.int8, device=dev_t)), T(torch.empty(M, device=dev_t))
            return lambda: ops.norm_quant(X, G1, 1e-6, None, Q, S, rot=A.ROT_SYLVESTER, group=128)
        return make
    run("cfg4_rmsnorm_wht128_quant_47104", make4(M4))

    # ---- config 5a: RMSNorm + modulate + int8 quant; 5b: int8 GEMM + dequant + SiLU ----
    sc5, sh5 = bf16(1, C, scale=0.5), bf16(1, C, scale=0.5)
    tb5 = ops.Tables(scale=T(sc5), shift=T(sh5))

    def make5a(M):
        def make():
            x = bf16(M, C)
            first.setdefault(f"x5_{M}", x)
            X, Q, S = T(x), T(torch.empty(M, C, dtype=torch.int8, device=dev_t)), T(torch.empty(M, device=dev_t))
            return lambda: ops.norm_quant(X, G1, 1e-6, tb5, Q, S)
        return make
    run("cfg5a_rmsnorm_mod_quant_47104", make5a(M4))
    # the GEMM's inputs: config 5a's codes and scales of the first set
    x5 = first.get(f"x5_{M4}", None)
    if x5 is None:
        x5 = bf16(M4, C)
    q5, s5 = torch.empty(M4, C, dtype=torch.int8, device=dev_t), torch.empty(M4, device=dev_t)
    Q5, S5 = T(q5), T(s5)
    ops.norm_quant(T(x5), G1, 1e-6, tb5, Q5, S5)
    w5 = torch.randint(-127, 128, (16384, C), dtype=torch.int8, device=dev_t)
    ws5 = (0.005 + 0.015 * torch.rand(16384, device=dev_t)).float()
    layer = ops.Int8Linear(T(w5), T(ws5))
    out5 = torch.empty(M4, 16384, dtype=torch.bfloat16, device=dev_t)
    O5 = T(out5)
    # the GEMM's output, the [gate | up] rows the MLP's middle reads: one untimed call here; the GEMM is timed after
    # every HBM-bound kernel, since a third of a second of it lowers the clock of the kernels timed right after it
    ops.int8_gemm_dequant(Q5, S5, layer, A.ACT_SILU, O5)

    # ---- the MLP's middle: swiglu of fc1's [gate | up] output [47104 x 2*8192] -> fc2's quantizer (regular g 256) ----
    def make6():
        q6, s6 = torch.empty(M4, 8192, dtype=torch.int8, device=dev_t), torch.empty(M4, device=dev_t)
        X6, Q6, S6 = O5, T(q6), T(s6)    # the GEMM's output rows are [gate | up] halves of 8192
        return lambda: ops.swiglu_quant(X6, Q6, S6, rot=A.ROT_REGULAR, group=256)
    run("mlp_swiglu_quant_g256_47104x8192", make6)

    # ---- configs 2-5a at the other token count: 47104 tokens (grid T46 x H32 x W32) for 2 and 3, 16896 for 4 and 5a ----
    def make2b():
        x, r, o = bf16(M4, C), bf16(M4, C), torch.empty(M4, C, dtype=torch.bfloat16, device=dev_t)
        X, R, O = T(x), T(r), T(o)
        return lambda: ops.norm_mod_act_gate(X, A.NORM_LAYER, None, None, 1e-5, tb2, A.ACT_GELU_TANH, R, O)
    run("cfg2_ln_mod_gelu_gate_47104", make2b)
    run("cfg3_qk_rmsnorm_rope3d_47104", make3(M4, T(torch.from_numpy(rope_table(46, 32, 32)).to(dev_t))))
    run("cfg4_rmsnorm_wht128_quant_16896", make4(M2))
    run("cfg5a_rmsnorm_mod_quant_16896", make5a(M2))

    # ---- the DiT block's bandwidth-bound calls, as the unchanged engine makes them (dit.rs:329-369), at 16896 and
    # 47104 tokens; each takes buffers of its own call shape (cache-cold rings as above) ----
    def dit_side(M):
        g = torch.Generator(device="cpu").manual_seed(M)
        rows = torch.zeros(M, dtype=torch.int32)
        rows[: M // 20] = 1                                      # engine/h3d/src/jobs.rs:213
        f32 = lambda *sh, sc=1.0, base=0.0: (base + sc * torch.randn(*sh, generator=g)).float().to(dev_t)   # noqa: E731
        side = {"rows": rows.to(dev_t), "w": f32(DH, sc=0.1, base=1.0), "scale": f32(2, DH, sc=0.1),
                "shift": f32(2, DH, sc=0.1), "gate": f32(2, DH, sc=0.5), "qn": f32(DHD, sc=0.1, base=1.0),
                "kn": f32(DHD, sc=0.1, base=1.0)}
        # (cos, sin) of the three position axes per token, 21 frequencies each (dit.rs:188-203)
        pos = torch.randint(0, 64, (M, 3), generator=g).float()
        inv = torch.pow(torch.tensor(10000.0), -torch.arange(21).float() / 21.0)
        ang = (pos[:, :, None] * inv[None, None, :]).reshape(M, 63)
        side["cs126"] = torch.stack([torch.cos(ang), torch.sin(ang)], -1).contiguous().to(dev_t)
        side["cs96"] = side["cs126"][:, :48].contiguous()
        return {k: T(v) for k, v in side.items()}

    def dit_hbm(M):
        sd = dit_side(M)
        mod = ops.Mod(sd["rows"], sd["scale"], sd["shift"])

        def norm():
            x, h = bf16(M, DH), torch.empty(M, DH, dtype=torch.bfloat16, device=dev_t)
            X, H = T(x), T(h)
            return lambda: ops.rms_norm_mod(X, sd["w"], 1e-5, mod, H)
        run(f"dit_rms_norm_mod_{M}", norm)

        def rope(part, w, rot, cs, both=False):
            def make():
                qkv = bf16(M, DQKV)
                QKV = T(qkv)
                r = [ops.Rows(QKV, i * DHEADS * DHD, DQKV, M, DHEADS, DHD) for i in range(2)]
                if both:
                    return lambda: ops.qk_rms_rope(r[0], r[1], sd["qn"], sd["kn"], 1e-5, cs, rot)
                return lambda: ops.rms_rope(r[part], w, 1e-5, cs, rot)
            return make
        run(f"dit_rms_rope_q_rot126_{M}", rope(0, sd["qn"], 126, sd["cs126"]))
        run(f"dit_rms_rope_k_rot126_{M}", rope(1, sd["kn"], 126, sd["cs126"]))
        run(f"dit_rms_rope_q_rot96_{M}", rope(0, sd["qn"], 96, sd["cs96"]))
        run(f"dit_qk_rms_rope_rot126_{M}", rope(0, None, 126, sd["cs126"], both=True))

        def gate_add():
            x, pr = bf16(M, DH), bf16(M, DH)
            X, PR = T(x), T(pr)
            return lambda: ops.gate_add(X, PR, sd["rows"], sd["gate"])
        run(f"dit_gate_add_{M}", gate_add)

        def swiglu():
            f1, act = bf16(M, 2 * DFF), torch.empty(M, DFF, dtype=torch.bfloat16, device=dev_t)
            F1, ACT = T(f1), T(act)
            return lambda: ops.swiglu(F1, ACT)
        run(f"dit_swiglu_{M}", swiglu)

        def quantize(K):
            def make():
                x = bf16(M, K)
                X, Q, S = T(x), T(torch.empty(M, K, dtype=torch.int8, device=dev_t)), T(torch.empty(M, device=dev_t))
                return lambda: ops.int8_quantize(X, Q, S, 256)
            return make
        for name, K, _ in DIT_LINEARS:
            if name != "fc1":                                    # fc1 quantizes the same h as qkv
                run(f"dit_quantize_g256_{name}_{M}", quantize(K))

        # the fused forms of the pairs dit.rs:340-341 and 363-364
        def norm_quant():
            x = bf16(M, DH)
            X, Q, S = T(x), T(torch.empty(M, DH, dtype=torch.int8, device=dev_t)), T(torch.empty(M, device=dev_t))
            tb = ops.Tables(scale=sd["scale"], shift=sd["shift"], rows=sd["rows"])
            return lambda: ops.norm_quant(X, sd["w"], 1e-5, tb, Q, S, rot=A.ROT_REGULAR, group=256)
        run(f"dit_norm_quant_g256_{M}", norm_quant)

        def swiglu_quant():
            f1 = bf16(M, 2 * DFF)
            F1, Q, S = T(f1), T(torch.empty(M, DFF, dtype=torch.int8, device=dev_t)), T(torch.empty(M, device=dev_t))
            return lambda: ops.swiglu_quant(F1, Q, S, rot=A.ROT_REGULAR, group=256)
        run(f"dit_swiglu_quant_g256_{M}", swiglu_quant)

    dit_hbm(M2)
    dit_hbm(M4)

    # torch's elementwise kernels with the fused kernels' traffic shapes (every run, before the compute-bound
    # kernels: the rate attainable for each shape)
    for M in (M2, M4):
        def make_add(M=M):
            x, r, o = bf16(M, C), bf16(M, C), torch.empty(M, C, dtype=torch.bfloat16, device=dev_t)
            return lambda: torch.add(x, r, out=o)
        run(f"probe_add_bf16_{M}x{C}", make_add)

        def make_halfadd(M=M):
            x, o = bf16(M, C), torch.empty(M, C // 2, dtype=torch.bfloat16, device=dev_t)
            a, b = x[:, : C // 2], x[:, C // 2:]
            return lambda: torch.add(a, b, out=o)
        run(f"probe_halfadd_bf16_{M}x{C}", make_halfadd)

        def make_inplace(M=M):
            qkv = bf16(M, 3 * 7168)
            q = qkv[:, :7168]
            return lambda: q.mul_(1.0)
        run(f"probe_inplace_bf16_{M}x7168_of_21504", make_inplace)

    # ---- the compute-bound kernels, last: config 5b's int8 GEMM, then attention ----
    run("cfg5b_int8_gemm_silu_47104x16384", lambda: (lambda: ops.int8_gemm_dequant(Q5, S5, layer, A.ACT_SILU, O5)), 5)

    # ---- attention of the 16896-token grid, 32 heads of 128 (the int8 form: S >= 8192), and at 47104 tokens ----
    def make_attn(M):
        def make():
            qkv, o = bf16(M, 3 * 4096), torch.empty(M, 4096, dtype=torch.bfloat16, device=dev_t)
            QKV, O = T(qkv), T(o)
            rows = [ops.Rows(QKV, i * 4096, 3 * 4096, M, 32, 128) for i in range(3)]
            return lambda: ops.attention(*rows, O)
        return make
    run("attn_sage_16896x32x128", make_attn(M2), 10)
    run("attn_sage_47104x32x128", make_attn(M4), 3)
    # the 16-bit form, which the reference takes below 8192 tokens: 4096 tokens x 32 heads x 128
    run("attn_f16_4096x32x128", make_attn(4096), 20)

    # ---- the DiT block's int8 linears (group 256, a scale per output) and its attention, 56 heads of 128 ----
    def dit_compute(M):
        gen = torch.Generator(device="cpu").manual_seed(M + 1)
        for name, K, N in DIT_LINEARS:
            key = f"dit_int8_linear_{name}_{M}"
            if skip(key):
                continue
            w = torch.randint(-127, 128, (N, K), dtype=torch.int8, generator=gen).to(dev_t)
            ws = (0.005 + 0.015 * torch.rand(N, generator=gen)).float().to(dev_t)
            lin = ops.Int8Linear(T(w), T(ws), group=256)
            x, out = bf16(M, K), torch.empty(M, N, dtype=torch.bfloat16, device=dev_t)
            X, O = T(x), T(out)
            run(key, lambda: (lambda: lin.forward(X, O)), 5, ring=1)
            del w, x, out, X, O, lin
            torch.cuda.empty_cache()

        def attn():
            qkv, o = bf16(M, DQKV), torch.empty(M, DHEADS * DHD, dtype=torch.bfloat16, device=dev_t)
            QKV, O = T(qkv), T(o)
            rows = [ops.Rows(QKV, i * DHEADS * DHD, DQKV, M, DHEADS, DHD) for i in range(3)]
            return lambda: ops.attention(*rows, O)
        run(f"dit_attention_{M}", attn, 5 if M < 30000 else 2, ring=1)

    dit_compute(M2)
    dit_compute(M4)

    # ---- the float linear on bfloat16 activations (h3s_linear, h3s_linear_acc) ----
    # (the LoRA factors stream their rows: cache-cold rings as above; the linear of the hidden width is
    # compute-bound: one buffer set)
    gen = torch.Generator(device="cpu").manual_seed(7)

    def make_fl(lin, Mf, K, N, acc):
        def make():
            X, O = T(bf16(Mf, K)), T(bf16(Mf, N))
            return (lambda: lin.forward_acc(X, O)) if acc else (lambda: lin.forward(X, O))
        return make
    for Mf in (M2, M4):
        for name, K, N, has_bias, acc in FLOAT_LINEARS:
            key = f"{name}_{Mf}x{K}x{N}"
            if skip(key) or key not in B:
                continue
            w = (torch.randn(N, K, generator=gen) / K ** 0.5).to(torch.bfloat16).to(dev_t)
            bias = (0.1 * torch.randn(N, generator=gen)).float().to(dev_t)
            lin = ops.Linear(T(w), T(bias) if has_bias else None)
            run(key, make_fl(lin, Mf, K, N, acc), 10, ring=None if name.startswith("lora_") else 1)
            del w, bias, lin
            torch.cuda.empty_cache()
    key = f"probe_matmul_bf16_{M2}x{DH}x{DH}"
    if not skip(key):
        w = (torch.randn(DH, DH, generator=gen) / DH ** 0.5).to(torch.bfloat16).to(dev_t)
        x, out = bf16(M2, DH), torch.empty(M2, DH, dtype=torch.bfloat16, device=dev_t)
        wt = w.t()
        run(key, lambda: (lambda: torch.matmul(x, wt, out=out)), 10, ring=1)
        del w, wt, x, out
        torch.cuda.empty_cache()

    if args.copy_probe:
        def make_copy():
            src = torch.empty(1 << 29, dtype=torch.bfloat16, device=dev_t).fill_(1.0)
            dst = torch.empty_like(src)
            return lambda: dst.copy_(src)
        run("copy_probe_1GiB", make_copy, 20)

        def make_copy1():
            src = torch.empty(CFG1_COPY_ELEMS, dtype=torch.bfloat16, device=dev_t).fill_(1.0)
            dst = torch.empty_like(src)
            return lambda: dst.copy_(src)
        run("copy_probe_cfg1_bytes", make_copy1, 200)


    per = {}
    for k, ms in kernels.items():
        gbs = B[k] / (ms * 1e-3) / 1e9
        e = {"ms": round(ms, 5), "ms_mean": round(means[k], 5), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_GBS, 4),
             "bytes": B[k], "ring": rings[k], "steps": steps_of[k]}
        if k.startswith("cfg5b"):
            tops = 2 * M4 * C * 16384 / (ms * 1e-3) / 1e12
            e.update({"TOPS_i8": round(tops, 1), "frac_i8_peak": round(tops / PEAK_I8_TOPS, 4)})
        if k.startswith("dit_int8_linear"):
            Mk = int(k.rsplit("_", 1)[1])
            K_, N_ = next((K, N) for name, K, N in DIT_LINEARS if k.startswith(f"dit_int8_linear_{name}_"))
            tops = 2 * Mk * K_ * N_ / (ms * 1e-3) / 1e12
            e.update({"TOPS_i8": round(tops, 1), "frac_i8_peak": round(tops / PEAK_I8_TOPS, 4)})
        m_fl = re.match(r"(linear_bf16|lora_a_bf16|lora_b_acc_bf16|probe_matmul_bf16)_(\d+)x(\d+)x(\d+)$", k)
        if m_fl:
            Mk, K_, N_ = (int(v) for v in m_fl.groups()[1:])
            tf = 2 * Mk * K_ * N_ / (ms * 1e-3) / 1e12
            e.update({"TFLOPS_bf16": round(tf, 1), "frac_bf16_peak": round(tf / PEAK_F16_TFLOPS, 4)})
        if k.startswith("dit_attention"):
            Mk = int(k.rsplit("_", 1)[1])
            half_ops = 2.0 * Mk * Mk * DHEADS * DHD
            t_peak = half_ops / (PEAK_I8_TOPS * 1e12) + half_ops / (PEAK_F16_TFLOPS * 1e12)
            e.update({"TOPS": round(2 * half_ops / (ms * 1e-3) / 1e12, 1), "frac_mfma_peak": round(t_peak / (ms * 1e-3), 4)})
        if k.startswith("attn"):
            # the int8 form: q k^T on the i8 cores (5 POPS) and P v on the f16 cores (2.5 PFLOP/s); the 16-bit form:
            # both on the f16 cores. The time both take at peak.
            S_ = int(re.search(r"_(\d+)x32x128", k).group(1))
            half_ops = 2.0 * S_ * S_ * 4096
            qk_peak = PEAK_F16_TFLOPS if k.startswith("attn_f16") else PEAK_I8_TOPS
            t_peak = half_ops / (qk_peak * 1e12) + half_ops / (PEAK_F16_TFLOPS * 1e12)
            e.update({"TOPS": round(2 * half_ops / (ms * 1e-3) / 1e12, 1), "frac_mfma_peak": round(t_peak / (ms * 1e-3), 4)})
        per[k] = e

    value = B[HEADLINE] / (ms2 * 1e-3) / 1e9
    line = {
        "metric": "achieved HBM GB/s (% of 8 TB/s) per fused kernel at 16.8k/47k tokens x 4096",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms2, 5),
        "ms_per_step_mean": round(means[HEADLINE], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (torch.randn on the device; shift/scale/gate ~N(0,0.5))",
        "config": {"workload": "AdaLN chain: LayerNorm(no affine) -> x*(1+scale)+shift -> GELU-tanh -> res + gate*y, "
                               "X,res [16896 x 4096] bf16 (grid T16xH24xW44), cache-cold: a ring of "
                               f"{n2} buffer sets ({n2 * B[HEADLINE] / 1e9:.2f} GB)", "tokens": M2, "hidden": C},
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / PEAK_GBS, 4), "traffic": measured_traffic(HEADLINE)},
        "kernels": per,
        "device": dev.name(),
        "library": os.path.relpath(A.load().path, ROOT),
        "cus": torch.cuda.get_device_properties(0).multi_processor_count,
    }
    dit = dit_block_table(kernels)
    if dit:
        line["dit_block"] = dit
    if args.mark:
        line["marked"] = marked
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(x2, r2, tab, {"x1": first["x1"], "g1": g1, "wq": wq, "wk": wk, "cs": cs,
                                                          "q3": first.get(f"q3_{M2}"), "k3": first.get(f"k3_{M2}"),
                                                          "x4": first.get(f"x4_{M4}"), "x5": x5, "sc5": sc5, "sh5": sh5,
                                                          "q5": q5, "s5": s5, "w5": w5, "ws5": ws5})
    print(json.dumps(line), flush=True)
    return 0


def dit_block_table(kernels: dict) -> dict:
    """The DiT block's time per stage under the labels of the reference's harness (engine/h3d/src/jobs.rs:269-279),
    each stage the sum of its calls' times (the norm and the gated add run twice a block), beside the engine's
    published times per block (docs/PORT-PLAN.md:62-70, on its own GPU); and the three fused pairs against the two
    calls each replaces."""
    out = {}
    for M in (M2, M4):
        st = {}
        for label, keys in DIT_STAGES:
            ks = [f"{k}_{M}" for k in keys]
            if all(k in kernels for k in ks):
                st[label] = round(sum(kernels[k] for k in ks), 4)
        if not st:
            continue
        e = {"stages_ms": st, "ms_per_block": round(sum(st.values()), 3) if len(st) == len(DIT_STAGES) else None}
        pairs = {
            "rms_norm_mod + int8_linear's quantizer (dit.rs:340-341) -> h3s_norm_quant":
                (("dit_rms_norm_mod", "dit_quantize_g256_qkv"), "dit_norm_quant_g256"),
            "swiglu + fc2's quantizer (dit.rs:363-364) -> h3s_swiglu_quant":
                (("dit_swiglu", "dit_quantize_g256_fc2"), "dit_swiglu_quant_g256"),
            "rms_rope of q + of k (dit.rs:347-348) -> h3s_qk_rms_rope": (("dit_rms_rope_q_rot126", "dit_rms_rope_k_rot126"),
                                                                         "dit_qk_rms_rope_rot126"),
        }
        fused = {}
        for label, (two, one) in pairs.items():
            ks, k1 = [f"{k}_{M}" for k in two], f"{one}_{M}"
            if all(k in kernels for k in ks) and k1 in kernels:
                fused[label] = {"two_calls_ms": round(sum(kernels[k] for k in ks), 4), "fused_ms": round(kernels[k1], 4)}
        if fused:
            e["fused_pairs"] = fused
        out[str(M)] = e
    if out:
        out["published_engine_ms_per_block"] = DIT_PUBLISHED_MS
    return out


def cpu_baseline(x2, r2, tab, t):
    """The CPU oracle (oracle/h3oracle.c, the C restatement of the reference arithmetic, row-parallel with contiguous
    row chunks as engine/h3-core/src/reference.rs:43-80) on this host, one thread per CPU of the process's share (the
    cgroup quota or affinity mask, at most 16: the host's share for one GPU): the headline workload in full, the median
    of the runs that fit about 10 s; under `kernels` the other configurations on the tensors the GPU ran (the GEMM on
    its first 1024 rows, scaled linearly), each the median of at least 5 runs."""
    import numpy as np
    import torch

    from oracle import oracle as o

    share = cpu_share()
    avail = min(share["affinity"], int(share["cgroup_quota"]) if share["cgroup_quota"] else share["affinity"])
    threads = max(1, min(16, avail))
    o.set_threads(threads)
    u16 = lambda a: a.view(torch.int16).cpu().numpy().view(np.uint16).ravel()   # noqa: E731
    f32 = lambda a: a.float().cpu().numpy().ravel()                              # noqa: E731

    def median_time(fn, budget, least=5, most=50):
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
    gbs = B[HEADLINE] / med / 1e9
    out = {"value": round(gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
           "sample": f"the full 16896 x 4096 workload, median of {n} runs ({med * 1e3:.1f} ms each), {threads} threads "
                     f"on {share['model']} (nproc {share['nproc']}, affinity {share['affinity']}, cgroup quota "
                     f"{share['cgroup_quota']}; at most 16 threads: the CPU share a one-GPU job has on these hosts, "
                     f"whatever nproc shows)",
           "host": share}

    per = {}
    x1, g1 = u16(t["x1"]), f32(t["g1"])
    per["cfg1_rmsnorm_quant_2159"] = median_time(lambda: o.norm_quant(x1, o.BF16, 2159, C, g1, 1e-6), 2.0)[0]
    if t["q3"] is not None:
        q3, k3, wq, wk, cs = u16(t["q3"]), u16(t["k3"]), f32(t["wq"]), f32(t["wk"]), f32(t["cs"])
        per["cfg3_qk_rmsnorm_rope3d_16896"] = median_time(lambda: (o.rms_rope(q3, o.BF16, M2, 32, 128, 4096, wq, 1e-5, cs, 128),
                                                                   o.rms_rope(k3, o.BF16, M2, 32, 128, 4096, wk, 1e-5, cs, 128)), 2.0)[0]
    if t["x4"] is not None:
        x4 = u16(t["x4"])
        per["cfg4_rmsnorm_wht128_quant_47104"] = median_time(
            lambda: o.norm_quant(x4, o.BF16, M4, C, g1, 1e-6, rot=o.ROT_SYLVESTER, group=128), 2.0)[0]
    x5, sc5, sh5 = u16(t["x5"]), u16(t["sc5"]), u16(t["sh5"])
    per["cfg5a_rmsnorm_mod_quant_47104"] = median_time(lambda: o.norm_quant(x5, o.BF16, M4, C, g1, 1e-6, None, sc5, sh5, o.BF16), 2.0)[0]
    rows = 1024
    q5 = t["q5"][:rows].cpu().numpy().ravel()
    s5 = t["s5"][:rows].cpu().numpy().ravel()
    w5, ws5 = t["w5"].cpu().numpy().ravel(), f32(t["ws5"])
    per["cfg5b_int8_gemm_silu_47104x16384"] = median_time(
        lambda: o.gemm_dequant(q5, s5, rows, C, w5, 16384, ws5, act=o.ACT_SILU), 2.0, least=5)[0] * M4 / rows
    kernels = {}
    for k, sec in per.items():
        e = {"ms": round(sec * 1e3, 3), "GB/s": round(B[k] / sec / 1e9, 2)}
        if k.startswith("cfg5b"):
            e["TOPS_i8"] = round(2 * M4 * C * 16384 / sec / 1e12, 3)
            e["sample"] = f"the first {rows} of {M4} rows, time scaled by {M4 / rows:.1f}"
        kernels[k] = e
    out["kernels"] = kernels
    return out


# ---- the profiles/ tables: a rocprofv3 csv of a --mark run, cut into the timed dispatches of each workload ----
def _short(name: str) -> str:
    return re.sub(r"\(.*", "", name).replace("void ", "").strip()


def _dispatches(path: str):
    """(dispatch id, kernel name, row) in launch order; counter csvs hold one row per counter and dispatch"""
    rows = list(csv.DictReader(open(path)))
    key = "Dispatch_Id" if rows and "Dispatch_Id" in rows[0] else "Correlation_Id"
    rows.sort(key=lambda r: int(r[key]))
    return key, rows


def _regions(rows, key, marked):
    """the dispatches between each pair of markers, keyed by the marked workloads in order"""
    out, cur, inside, i, seen = {}, [], False, 0, set()
    for r in rows:
        d = r[key]
        if MARKER in r["Kernel_Name"]:
            if d in seen:
                continue
            seen.add(d)
            if inside:
                if i < len(marked):
                    out[marked[i]] = cur
                i += 1
            cur, inside = [], not inside
            continue
        if inside:
            cur.append(r)
    return out


def _bench(path):
    if not path:
        return {}
    txt = open(path).read().strip().splitlines()
    return json.loads([l for l in txt if l.startswith("{")][-1])


def summarize_trace(path: str, bench_json: str) -> str:
    """Markdown: per workload, its kernels' mean and median rocprofv3 durations over exactly the timed launches,
    against bench.py's HIP-event time per launch of the same run."""
    b = _bench(bench_json)
    key, rows = _dispatches(path)
    regions = _regions(rows, key, b.get("marked", []))
    lines = ["| workload | kernel | dispatches | mean µs | median µs | µs per launch (all its kernels) | bench µs per launch (HIP events) | ratio |",
             "|---|---|---:|---:|---:|---:|---:|---:|"]
    for w, rs in regions.items():
        steps = b.get("kernels", {}).get(w, {}).get("steps")
        per_kernel = collections.OrderedDict()
        for r in rs:
            per_kernel.setdefault(_short(r["Kernel_Name"]), []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        bench_us = b["kernels"][w]["ms"] * 1e3 if w in b.get("kernels", {}) else float("nan")
        first_k = next(iter(per_kernel.values()), [])
        launches = steps or len(first_k) or 1
        total = sum(sum(v) for v in per_kernel.values()) / launches
        for j, (kn, v) in enumerate(per_kernel.items()):
            v_sorted = sorted(v)
            med = v_sorted[len(v) // 2]
            tail = (f"{total:.2f} | {bench_us:.2f} | {total / bench_us:.3f}" if j == 0 else " | | ")
            lines.append(f"| {w if j == 0 else ''} | `{kn}` | {len(v)} | {sum(v) / len(v):.2f} | {med:.2f} | {tail} |")
    return "\n".join(lines)


def summarize_pmc(paths, bench_json: str) -> str:
    """Markdown: per workload, each counter summed over a launch's dispatches and averaged over the timed launches.
    With FETCH_SIZE and WRITE_SIZE and the --copy-probe region: the HBM traffic per launch, each counter scaled by what
    it reads for the 1 GiB copy, against the algorithmic bytes, and one machine-readable `traffic:` line per workload
    (read by bench.py's roofline.traffic). With SQ_VALU_MFMA_BUSY_CYCLES and GRBM_GUI_ACTIVE: the matrix cores' busy
    fraction, busy / (GRBM_GUI_ACTIVE x CUs x 4 SIMDs)."""
    b = _bench(bench_json)
    cus = int(b.get("cus", 256))
    vals = collections.defaultdict(lambda: collections.defaultdict(float))   # workload -> counter -> sum
    names = collections.defaultdict(set)
    span = collections.defaultdict(dict)                                     # workload -> dispatch -> duration ns
    for path in paths:
        key, rows = _dispatches(path)
        for w, rs in _regions(rows, key, b.get("marked", [])).items():
            for r in rs:
                vals[w][r["Counter_Name"]] += float(r["Counter_Value"])
                names[w].add(_short(r["Kernel_Name"]))
                if "Start_Timestamp" in r:
                    span[w][r[key]] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    B = bytes_cfg()
    counters = sorted({c for w in vals for c in vals[w]})
    lines = ["| workload | kernels | " + " | ".join(f"{c} per launch" for c in counters) + " |",
             "|---|---|" + "---:|" * len(counters)]
    per_launch, dur = {}, {}
    for w in vals:
        n = b["kernels"][w]["steps"]
        if span[w]:
            dur[w] = sum(span[w].values()) / n
        per_launch[w] = {c: vals[w][c] / n for c in vals[w]}
        lines.append(f"| {w} | {', '.join('`' + k + '`' for k in sorted(names[w]))} | " +
                     " | ".join(f"{per_launch[w].get(c, float('nan')):.1f}" for c in counters) + " |")
    out = "\n".join(lines)
    cal = per_launch.get("copy_probe_1GiB", {})
    if "FETCH_SIZE" in counters and "WRITE_SIZE" in counters and cal.get("FETCH_SIZE") and cal.get("WRITE_SIZE"):
        kib = (1 << 30) / 1024.0
        sf, sw = kib / cal["FETCH_SIZE"], kib / cal["WRITE_SIZE"]
        t = [f"\nCalibration (the 1 GiB device copy: {kib:.0f} KiB read and written): FETCH_SIZE reads "
             f"{cal['FETCH_SIZE']:.1f} KiB, scale {sf:.3f}; WRITE_SIZE reads {cal['WRITE_SIZE']:.1f} KiB, scale {sw:.3f}.\n",
             "| workload | scaled fetch + write bytes per launch | algorithmic bytes | ratio |", "|---|---:|---:|---:|"]
        mr = []
        for w in vals:
            if w == "copy_probe_1GiB" or w not in B:
                continue
            tb = int(round((per_launch[w].get("FETCH_SIZE", 0) * sf + per_launch[w].get("WRITE_SIZE", 0) * sw) * 1024))
            t.append(f"| {w} | {tb:,} | {B[w]:,} | {tb / B[w]:.4f} |")
            mr.append(f"traffic: {w} bytes={tb} algorithmic={B[w]}")
        out += "\n" + "\n".join(t) + "\n\n" + "\n".join(mr)
    if "SQ_VALU_MFMA_BUSY_CYCLES" in counters and "GRBM_GUI_ACTIVE" in counters:
        # GRBM_GUI_ACTIVE counts the busy cycles of each XCD's graphics block, summed over the XCDs: divided by them it
        # is the kernel's length in cycles (its quotient by the dispatch's duration is the clock, shown as a check).
        # SQ_VALU_MFMA_BUSY_CYCLES is summed over every SIMD: divided by the SIMDs and the kernel's cycles it is the
        # fraction of time a SIMD's matrix core is busy.
        xcds = int(b.get("xcds", 8))
        t = [f"\n| workload | kernel cycles (GRBM_GUI_ACTIVE / {xcds} XCDs) | clock GHz | MFMA busy per SIMD "
             f"(SQ_VALU_MFMA_BUSY_CYCLES / ({cus} CUs x 4 SIMDs x kernel cycles)) |", "|---|---:|---:|---:|"]
        for w in vals:
            g = per_launch[w].get("GRBM_GUI_ACTIVE", 0) / xcds
            if g:
                ns = dur.get(w)
                ghz = f"{g / ns:.2f}" if ns else "n/a"
                t.append(f"| {w} | {g:,.0f} | {ghz} | {per_launch[w]['SQ_VALU_MFMA_BUSY_CYCLES'] / (g * cus * 4):.4f} |")
        out += "\n" + "\n".join(t)
    if {"SQ_INSTS_VALU", "SQ_ACTIVE_INST_VALU", "SQ_WAVES", "GRBM_GUI_ACTIVE"} <= set(counters):
        # VALU issue: instructions per wavefront, and the profiler's VALUBusy for gfx950,
        # SQ_ACTIVE_INST_VALU / (CUs x kernel cycles): near or above 1 the kernel is bound by VALU issue, not by HBM
        xcds = int(b.get("xcds", 8))
        t = [f"\n| workload | wavefronts | VALU instructions per wavefront | VALU busy (SQ_ACTIVE_INST_VALU / ({cus} CUs x "
             f"GRBM_GUI_ACTIVE / {xcds})) |", "|---|---:|---:|---:|"]
        for w in vals:
            pl = per_launch[w]
            g = pl.get("GRBM_GUI_ACTIVE", 0) / xcds
            if g and pl.get("SQ_WAVES"):
                t.append(f"| {w} | {pl['SQ_WAVES']:,.0f} | {pl['SQ_INSTS_VALU'] / pl['SQ_WAVES']:,.0f} | "
                         f"{pl['SQ_ACTIVE_INST_VALU'] / (cus * g):.3f} |")
        out += "\n" + "\n".join(t)
    return out


if __name__ == "__main__":
    sys.exit(main())
