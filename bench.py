"""Benchmark: LoRA fwd + fused CE + bwd + AdamW tokens/s on one MI355X.

Default workload is config C2 of BASELINE.json: Qwen3-1.7B (28 layers, random
fp16 frozen weights N(0, 0.02), norms 1), rank-16 LoRA on Q/K/V/O, batch 1,
seq 128, token ids uniform over the vocabulary, next-token targets.  The step
runs as one captured HIP graph of libllmt.so kernels (llmt_step); inputs are
resident in HBM before the timed region.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c1|c2|c3|c4] [--only] [--no-cpu]
    python bench.py --copy-cal      # plain 512 MiB copies (PMC byte-counter scale)

Prints ONE JSON line.  Besides the contract fields it carries
  roofline:     the frozen-weight GEMMs (the step's dominant kernel family),
                each GEMM kind of the step replayed back to back as a HIP
                graph of its own (llmt_profile_kernels), timed with HIP
                events on the context's stream; achieved = streamed weight
                bytes per launch / average launch time, against 8 TB/s HBM
                (C4: TFLOP/s against 2.5 PFLOP/s); attainable_frac = the
                launches' roofline times (max of MFMA time at peak and
                compulsory HBM time) over their measured times; traffic =
                measured HBM bytes per launch (rocprofv3 FETCH_SIZE and
                WRITE_SIZE passes scaled by the copy calibration, read from
                profiles/gemm_<config>_traffic.md);
  roofline_bwd: the same for the backward's dX GEMMs alone (the metric's
                "bwd % MFMA / HBM peak"): hbm_frac and mfma_frac both given;
  kernels:      per-category kernel milliseconds of a step from the same
                replays (kernels only: their sum, kernels_sum_ms, is below
                ms_per_step by the launch gaps);
  bandwidth_kernels: AdamW, SwiGLU backward, RMSNorm backward and the fused
                CE in GB/s of their compulsory bytes, with frac of the
                datasheet 8 TB/s and copy_frac of the device copy rate
                (copy_gbs) measured in the same run;
  cpu_baseline: the CPU oracle (PyTorch fp32, oracle/lora_step.py) on a
                bounded sample of the same step (c4, c3 and c1 carry their own);
  c4, c3, c1:   (default run) the C4 step (B8 x S512, int8 weights), the
                C3 attention block and the C1 head (lm_head + CE + dX)
                measured in the same run; the C4 GEMM roofline also as
                frac_of_hipblaslt, against the 8192^3 fp16 hipBLASLt GEMM
                of the same run (achievable.mfma_f16_tflops_hipblaslt).
--config c1 / c3 / c4 --only times one of those alone; --kinds-md also prints the
per-kind markdown table of the step (the profiles/ kind tables).
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT), str(ROOT / "llm.cu_amd"), str(ROOT / "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "LoRA fwd+bwd+AdamW tokens/s, Qwen3-1.7B seq=128; bwd % MFMA / HBM peak"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0


def build_model(ctx, dims, seed, dev, int8=False):
    """Random frozen weights generated on the device, layer by layer."""
    import torch
    import llmt
    g = torch.Generator(device=dev).manual_seed(seed)
    H, Q, KV, I = dims.hidden, dims.n_heads * dims.head_dim, dims.n_kv_heads * dims.head_dim, \
        dims.intermediate
    ones = lambda n: torch.ones(n, dtype=torch.float32, device=dev)
    shapes = [(Q, H), (KV, H), (KV, H), (H, Q), (I, H), (I, H), (H, I)]
    for l in range(dims.n_layers):
        ws = [(torch.randn(s, generator=g, device=dev) * 0.02) for s in shapes]
        if int8:
            qs, scs = [], []
            for w in ws:
                q, s = llmt.quantize_rows_i8(w)
                qs.append(q)
                scs.append(s.half())
            ctx.set_layer_i8(l, qs, scs, ones(H), ones(H), ones(dims.head_dim),
                             ones(dims.head_dim))
        else:
            ctx.set_layer_f16(l, *[w.half() for w in ws], ones(H), ones(H), ones(dims.head_dim),
                              ones(dims.head_dim))
        del ws
    E = (torch.randn(dims.vocab, H, generator=g, device=dev) * 0.02).half()
    ctx.set_embed_f16(E, ones(H))
    del E
    torch.cuda.synchronize()


def cpu_baseline_sampled(batch, seq_len):
    """For configurations too large to run whole on the CPU (C4): the CPU
    oracle step on 1-layer and 2-layer models of the same width, batch and
    sequence; per-layer = t2 - t1, head = t1 - per-layer, and the full step is
    extrapolated as head + n_layers x per-layer."""
    import torch
    from oracle import lora_step as ref
    from oracle.configs import make_adapters, make_model
    dims = ref.QWEN3_1_7B
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    t = {}
    for nl in (1, 2):
        d = ref.Dims(**{**dims.__dict__, "n_layers": nl})
        g = torch.Generator().manual_seed(4242)
        W, ad = make_model(g, d), make_adapters(g, d)
        win = torch.randint(0, d.vocab, (batch, seq_len + 1), generator=g, dtype=torch.int32)
        t0 = time.perf_counter()
        ref.train_step(W, ad, win[:, :-1], win[:, 1:], d, step=1)
        t[nl] = time.perf_counter() - t0
        del W, ad
    layer = max(t[2] - t[1], 1e-9)
    head = max(t[1] - layer, 0.0)
    total = head + dims.n_layers * layer
    return {
        "value": round(batch * seq_len / total, 3),
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"CPU oracle (PyTorch fp32) LoRA step on 1- and 2-layer models at "
                   f"B{batch}xS{seq_len} ({t[1]:.1f} s, {t[2]:.1f} s, one step each); full "
                   f"{dims.n_layers}-layer step extrapolated = head + {dims.n_layers} x layer = "
                   f"{total:.1f} s; {torch.get_num_threads()} threads on {cpu_description()}"),
    }


def cpu_baseline(batch, seq_len, min_s=10.0):
    """The CPU oracle (PyTorch fp32, oracle/lora_step.py) running the same
    step -- forward, fused CE, closed-form backward, AdamW -- on the same
    configuration with its own seeded random model: one warm-up step, then
    timed steps until about min_s seconds have passed (at least 3); the
    median step time gives tokens/s."""
    import torch
    from oracle import lora_step as ref
    from oracle.configs import make_adapters, make_model
    dims = ref.QWEN3_1_7B
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    g = torch.Generator().manual_seed(4242)
    W = make_model(g, dims)
    ad = make_adapters(g, dims)
    win = torch.randint(0, dims.vocab, (batch, seq_len + 1), generator=g, dtype=torch.int32)
    tok, tgt = win[:, :-1], win[:, 1:]
    ref.train_step(W, ad, tok, tgt, dims, step=1)
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < min_s and len(times) < 50):
        t0 = time.perf_counter()
        ref.train_step(W, ad, tok, tgt, dims, step=len(times) + 2)
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    return {
        "value": round(batch * seq_len / med, 3),
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"CPU oracle (PyTorch fp32, oracle/lora_step.py) full {dims.n_layers}-layer "
                   f"LoRA step (fwd + CE + bwd + AdamW) at B{batch}xS{seq_len}, random model; "
                   f"median of {len(times)} timed steps after 1 warm-up: {med:.3f} s/step; "
                   f"{torch.get_num_threads()} threads on {cpu_description()}"),
    }


def cpu_baseline_c3(B=1, S=2048, nq=16, nkv=8, min_s=10.0):
    """C3 on the CPU oracle (PyTorch fp32): QK-RMSNorm + RoPE, causal GQA
    attention forward and backward, the norm / RoPE backward, on a bounded
    sample (B1 x S2048: a quarter of the B4 workload), timed like
    cpu_baseline."""
    import torch
    from oracle import lora_step as ref
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    g = torch.Generator().manual_seed(1003)
    q, k, v, do = (torch.randn(B, S, h, 128, generator=g) for h in (nq, nkv, nkv, nq))
    w = torch.ones(128)
    cos, sin = ref.rope_tables(S, 128, 1e6)

    def run():
        qn = ref.rope_fwd(ref.rmsnorm(q, w, 1e-6), cos, sin)
        kn = ref.rope_fwd(ref.rmsnorm(k, w, 1e-6), cos, sin)
        o, lse = ref.attention_fwd(qn, kn, v)
        dq, dk, dv = ref.attention_bwd(do, qn, kn, v, o, lse)
        ref.rmsnorm_bwd(ref.rope_bwd(dq, cos, sin), q, w, 1e-6)
        ref.rmsnorm_bwd(ref.rope_bwd(dk, cos, sin), k, w, 1e-6)
    med, n = _timed_median(run, min_s)
    return {"value": round(B * S / med, 2), "unit": "tokens/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": (f"CPU oracle (PyTorch fp32) attention block fwd+bwd (QK-norm, RoPE, causal "
                       f"GQA {nq}/{nkv} heads) at B{B}xS{S} (a quarter of the B4 workload): "
                       f"median of {n} calls after 1 warm-up, {med:.3f} s/call; "
                       f"{torch.get_num_threads()} threads on {cpu_description()}")}


def cpu_baseline_c1(T=128, H=2048, V=151936, min_s=10.0):
    """C1 on the CPU oracle (PyTorch fp32): logits = hidden W^T, the fused
    cross entropy with dlogits, dhidden = dlogits W, on the whole workload."""
    import torch
    from oracle import lora_step as ref
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    g = torch.Generator().manual_seed(1001)
    W = torch.randn(V, H, generator=g) * 0.02
    x = torch.randn(T, H, generator=g)
    tgt = torch.randint(0, V, (T,), generator=g, dtype=torch.int32)
    valid = ref.valid_rows(1, T)

    def run():
        logits = x @ W.t()
        _, dlogits, _ = ref.cross_entropy(logits, tgt, valid)
        dlogits @ W
    med, n = _timed_median(run, min_s)
    return {"value": round(T / med, 2), "unit": "tokens/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": (f"CPU oracle (PyTorch fp32) lm_head GEMM + fused CE + dX GEMM at T{T}, "
                       f"V {V}, H {H} (the whole workload): median of {n} calls after 1 "
                       f"warm-up, {med:.3f} s/call; {torch.get_num_threads()} threads on "
                       f"{cpu_description()}")}


def _timed_median(fn, min_s):
    """One warm-up call, then calls until about min_s seconds (at least 3, at
    most 50): the median call time and the number of timed calls."""
    fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < min_s and len(times) < 50):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2], len(times)


def measured_traffic(name, key="traffic_bytes_per_launch"):
    """HBM bytes per launch from a committed rocprofv3 counter summary
    (profiles/<name>.md, the line `<key>: N`; None if absent)."""
    f = ROOT / "profiles" / f"{name}.md"
    if not f.exists():
        return None
    m = re.search(re.escape(key) + r":\s*(\d+)", f.read_text())
    return int(m.group(1)) if m else None


def achievable_peaks():
    """Measured ceilings on this GPU, reported beside the datasheet peaks: a
    1 GiB device copy (read + write bytes / time) and an 8192^3 fp16 GEMM
    through torch.mm (hipBLASLt)."""
    import torch
    src = torch.ones(256 << 20, device="cuda")
    dst = torch.empty_like(src)
    a = torch.randn(8192, 8192, device="cuda").half()
    b = torch.randn(8192, 8192, device="cuda").half()

    def timed(fn, n):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n

    t_copy = timed(lambda: dst.copy_(src), 10)
    t_mm = timed(lambda: torch.mm(a, b), 10)
    out = {"hbm_copy_gbs": round(2 * src.numel() * 4 / t_copy / 1e9, 1),
           "mfma_f16_tflops_hipblaslt": round(2 * 8192 ** 3 / t_mm / 1e12, 1),
           "datasheet": {"hbm_gbs": HBM_PEAK_GBS, "mfma_f16_tflops": MFMA_F16_PEAK_TFLOPS}}
    del src, dst, a, b
    torch.cuda.empty_cache()
    return out


def cpu_description():
    """CPU model, sockets and cores of the host (from /proc/cpuinfo)."""
    model, phys, cores = "unknown", set(), set()
    try:
        cur = {}
        for line in open("/proc/cpuinfo"):
            if ":" not in line:
                if cur:
                    phys.add(cur.get("physical id"))
                    cores.add((cur.get("physical id"), cur.get("core id")))
                cur = {}
                continue
            k, v = (x.strip() for x in line.split(":", 1))
            cur[k] = v
            if k == "model name":
                model = v
    except OSError:
        pass
    return f"{model}; {len(phys)} socket(s), {len(cores)} physical cores on the host"


def copy_calibration():
    """Three plain device copies of 512 MiB: what FETCH_SIZE / WRITE_SIZE read
    for a kernel of known traffic (the scale applied to the GEMM passes)."""
    import torch
    n = 128 << 20
    src = torch.ones(n, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration": {"bytes_read": n * 4, "bytes_written": n * 4,
                                           "copies": 3}}), flush=True)


def bench_c3(steps, warmup):
    """C3: QK-norm + RoPE + causal GQA attention forward and backward through
    llmt_attention_block_bwd (fp16 q/k/v/dO, fp32 gradients), B4 x S2048,
    16 query / 8 KV heads.  Work = 7 causal S x S x 128 products per (batch,
    query head): forward QK^T, PV; backward recomputed QK^T, dO V^T, P^T dO,
    dS^T Q, dS K."""
    import torch
    import llmt
    B, S, nq, nkv = 4, 2048, 16, 8
    g = torch.Generator(device="cuda").manual_seed(1003)
    rnd = lambda h: torch.randn(B, S, h, 128, generator=g, device="cuda").half()
    q, k, v, do = rnd(nq), rnd(nkv), rnd(nkv), rnd(nq)
    one = torch.ones(128, device="cuda")
    run = lambda: llmt.attention_block_bwd(q, k, v, one, one, do)
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        run()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    flops = 7 * B * nq * (S * (S + 1) / 2) * 128 * 2
    tf = flops / dt / 1e12
    return {
        "metric": "attention fwd+bwd (QK-norm, RoPE, causal GQA) tokens/s",
        "value": round(B * S / dt, 2), "unit": "tokens/s", "steps": steps, "warmup": warmup,
        "ms_per_step": round(dt * 1e3, 4),
        "workload": "C3: causal GQA attention block fwd+bwd, B4 x S2048, 16 Q / 8 KV heads, "
                    "head_dim 128, QK-norm, RoPE 1e6",
        "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": MFMA_F16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                     "traffic": measured_traffic("attention_c3_traffic",
                                                 "traffic_bytes_per_call"),
                     "kernel": "attention block (norm/RoPE + flash fwd + flash bwd)"},
    }


def bench_c1(steps, warmup):
    """C1: the fused cross-entropy + lm_head backward alone (llmt_head_ce on a
    context whose tied embedding is packed once): logits = hidden W^T,
    softmax + NLL + fp32 dlogits over V = 151936, dhidden = dlogits W, one
    host sync a call for the loss.  hidden fp16 N(0,1) [128, 2048], W fp16
    N(0,0.02), targets uniform.  Algorithmic bytes: W read twice (2 x 622.3
    MB fp16) + logits read and fp32 dlogits written (155.6 MB)."""
    import torch
    import llmt
    T, H, V = 128, 2048, 151936
    d = llmt.qwen3_dims()
    d.n_layers = 1
    ctx = llmt.Context(d, 1, T)
    g = torch.Generator(device="cuda").manual_seed(1001)
    W = (torch.randn(V, H, generator=g, device="cuda") * 0.02).half()
    ctx.set_embed_f16(W, torch.ones(H, device="cuda"))
    del W
    x = torch.randn(T, H, generator=g, device="cuda").half()
    tgt = torch.randint(0, V, (T,), generator=g, device="cuda", dtype=torch.int32)
    for _ in range(warmup):
        ctx.head_ce(x, tgt, want_dlogits=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        loss, _, _ = ctx.head_ce(x, tgt, want_dlogits=True)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    ctx.close()
    nbytes = 2 * V * H * 2 + 2 * T * V * 4
    gbs = nbytes / dt / 1e9
    return {
        "workload": "C1: fused CE + lm_head backward, hidden 128 x 2048 fp16, tied W 151936 x "
                    "2048 fp16, fp32 dlogits and dhidden (one host sync a call)",
        "value": round(T / dt, 2), "unit": "tokens/s", "steps": steps, "warmup": warmup,
        "ms_per_step": round(dt * 1e3, 4), "loss": round(loss, 5),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("head_c1_traffic", "traffic_bytes_per_call"),
                     "algorithmic_bytes": nbytes,
                     "kernel": "logits GEMM + fused CE + dX GEMM (whole call)"},
    }


def kernel_summary(kinds):
    """Per-category milliseconds per step from llmt_profile_kernels' per-kind
    replays (kernels only: no events between kernels, no launch gaps)."""
    import llmt
    cats = {c: 0.0 for c in llmt.PROFILE_CATEGORIES}
    for k in kinds:
        cats[k["category"]] += k["us"] * k["launches"] / 1e3
    return {c: round(v, 4) for c, v in cats.items()}


GEMM_SHAPE = re.compile(r"M(\d+) N(\d+) K(\d+)")


def gemm_attainable_us(k):
    """The roofline time of one GEMM launch: the larger of its MFMA time at
    the dense fp16 peak and its compulsory HBM time at 8 TB/s (the weights it
    streams, its fp16 A operand and its fp32 output, M x N x 4)."""
    M, N, K = (int(x) for x in GEMM_SHAPE.search(k["name"]).groups())
    hbm = k["bytes"] + M * K * 2 + M * N * 4
    return max(k["flops"] / (MFMA_F16_PEAK_TFLOPS * 1e12), hbm / (HBM_PEAK_GBS * 1e9)) * 1e6


def is_backward_gemm(k):
    """The dX GEMMs of the backward: the layers' and the lm_head's (K = V)."""
    if k["category"] == "gemm_bwd":
        return True
    m = GEMM_SHAPE.search(k["name"])
    return k["category"] == "gemm_lm_head" and m and int(m.group(3)) > int(m.group(2))


def gemm_family(kinds, pred=None):
    """A set of the step's frozen-weight GEMMs as one family: launches,
    average launch duration, algorithmic weight bytes and FLOPs per launch,
    and the fraction of the attainable roofline (sum of the launches'
    roofline times over their measured times)."""
    g = [k for k in kinds if k["category"] in ("gemm_fwd", "gemm_bwd", "gemm_lm_head")
         and (pred is None or pred(k))]
    n = sum(k["launches"] for k in g)
    t_us = sum(k["us"] * k["launches"] for k in g)
    by = sum(k["bytes"] * k["launches"] for k in g)
    fl = sum(k["flops"] * k["launches"] for k in g)
    att = sum(gemm_attainable_us(k) * k["launches"] for k in g)
    return n, t_us / n, by / n, fl / n, att / t_us


def roofline_obj(cfg, kinds, pred, label):
    """The roofline object of a GEMM family (see gemm_family)."""
    n, avg_us, bytes_per_launch, flops_per_launch, att = gemm_family(kinds, pred)
    gbs = bytes_per_launch / (avg_us * 1e-6) / 1e9
    tflops = flops_per_launch / (avg_us * 1e-6) / 1e12
    if cfg == "c2":  # intensity ~T = 128 flop/byte < ridge ~312: HBM-bound
        bound, ach, peak, unit = "hbm", round(gbs, 1), HBM_PEAK_GBS, "GB/s"
    else:            # T = 4096: MFMA-bound
        bound, ach, peak, unit = "mfma", round(tflops, 2), MFMA_F16_PEAK_TFLOPS, "TFLOP/s"
    sel = [k for k in kinds if k["category"].startswith("gemm") and (pred is None or pred(k))]
    return {
        "bound": bound,
        "kernel": label + " (" + ", ".join(sorted({k["name"].split()[0] for k in sel})) + ")",
        "achieved": ach, "peak": peak, "unit": unit, "frac": round(ach / peak, 4),
        "algorithmic_bytes_per_launch": round(bytes_per_launch),
        "launches_per_step": n,
        "avg_launch_us": round(avg_us, 3),
        "weight_gbs": round(gbs, 1),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "gemm_tflops": round(tflops, 2),
        "mfma_frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
        "attainable_frac": round(att, 4),
    }


def kinds_markdown(cfg, kinds):
    """Every kernel kind of one step as a markdown table: launches, average
    replayed launch duration, algorithmic work and rate, the bound and the
    fraction of it (GEMMs also against their attainable roofline time)."""
    lines = ["| Kind | Category | Launches | Avg us | Step ms | Work / launch | Rate | Bound | "
             "Frac of peak |", "|---|---|---:|---:|---:|---:|---:|---|---:|"]
    for k in sorted(kinds, key=lambda k: -k["us"] * k["launches"]):
        us, step_ms = k["us"], k["us"] * k["launches"] / 1e3
        if k["category"].startswith("gemm"):
            gbs = k["bytes"] / (us * 1e-6) / 1e9
            tf = k["flops"] / (us * 1e-6) / 1e12
            if cfg == "c2":
                work, rate = f"{k['bytes'] / 1e6:.2f} MB weights", f"{gbs:.0f} GB/s ({tf:.0f} TFLOP/s)"
                bound, frac = "HBM", gbs / HBM_PEAK_GBS
            else:
                work, rate = f"{k['flops'] / 1e9:.1f} GFLOP", f"{tf:.0f} TFLOP/s"
                bound, frac = "MFMA", tf / MFMA_F16_PEAK_TFLOPS
            bound += f"; attainable {gemm_attainable_us(k) / us:.0%}"
        elif k["flops"] > 0:
            tf = k["flops"] / (us * 1e-6) / 1e12
            work, rate, bound, frac = f"{k['flops'] / 1e9:.2f} GFLOP", f"{tf:.0f} TFLOP/s", \
                "MFMA", tf / MFMA_F16_PEAK_TFLOPS
        else:
            gbs = k["bytes"] / (us * 1e-6) / 1e9
            work, rate, bound, frac = f"{k['bytes'] / 1e6:.2f} MB", f"{gbs:.0f} GB/s", "HBM", \
                gbs / HBM_PEAK_GBS
        lines.append(f"| `{k['name']}` | {k['category']} | {k['launches']} | {us:.2f} | "
                     f"{step_ms:.3f} | {work} | {rate} | {bound} | {frac:.1%} |")
    total = sum(k["us"] * k["launches"] for k in kinds) / 1e3
    lines.append(f"\nSum of the kinds: {total:.3f} ms a step, "
                 f"{sum(k['launches'] for k in kinds)} launches.")
    return "\n".join(lines)


BANDWIDTH_KINDS = ("adamw", "swiglu_bwd", "norm_bwd", "cross_entropy")


def bandwidth_kernels(kinds):
    """The bandwidth-bound kernels of the step (north star: >= 70% of HBM):
    each kernel's bytes per launch as the library records them
    (llmt_profile_kernels: what the kernel's interface reads and writes in
    the dtypes it uses, split-K partials included), divided by its average
    replayed launch duration.
      adamw          p, g, m, v read and p, m, v written, fp32, per parameter,
                     and the two fp16 operand copies of the new value the
                     next step's GEMMs read (7 x 4 B + 2 x 2 B);
      swiglu_bwd     the down dX GEMM's fp32 split partials [split, T, I],
                     gate and up [T, 2I] fp16 read, dgate | dup [T, 2I] fp16
                     written;
      norm_bwd       the gate/up dX GEMM's split partials, x and the residual
                     gradient [T, H] fp32 read, the residual gradient fp32 and
                     the fp16 GEMM operand written;
      cross_entropy  the per-tile softmax pairs and the logits [T, V] fp32
                     read once, the fp16 dlogits operand [T, V] written."""
    out = {}
    for k in kinds:
        if k["name"] in BANDWIDTH_KINDS:
            b = k["bytes"]
            gbs = b / (k["us"] * 1e-6) / 1e9
            out[k["name"]] = {"us": round(k["us"], 2), "bytes": round(b), "gbs": round(gbs, 1),
                              "frac": round(gbs / HBM_PEAK_GBS, 4)}
    return out


def bench_step(cfg, steps, warmup, graph=True, kinds_md=False):
    """The LoRA training step of config c2 or c4 through llmt_step (one HIP
    graph launch a step), then llmt_profile_kernels for the per-kernel
    breakdown and the GEMM roofline."""
    import torch
    import llmt
    dev = torch.device("cuda:0")
    dims = llmt.qwen3_dims()
    if cfg == "c2":
        batch, seq_len, int8, seed = 1, 128, False, 1002
        workload = ("C2: Qwen3-1.7B LoRA training step (28 layers, fp16 frozen weights, rank-16 "
                    "Q/K/V/O adapters, fwd + fused CE + bwd + AdamW), batch 1 x seq 128")
    else:
        batch, seq_len, int8, seed = 8, 512, True, 1004
        workload = ("C4: Qwen3-1.7B LoRA training step (28 layers, int8 per-channel frozen "
                    "weights, fused dequant), batch 8 x seq 512")
    T = batch * seq_len
    ctx = llmt.Context(dims, max_batch=batch, seq_len=seq_len, int8=int8)
    build_model(ctx, dims, seed, dev, int8=int8)
    ctx.lora_init(seed, 1.0 / 2048 ** 0.5, 0.01)
    g = torch.Generator(device=dev).manual_seed(seed + 1)
    win = torch.randint(0, dims.vocab, (batch, seq_len + 1), generator=g, device=dev,
                        dtype=torch.int32)
    tok, tgt = win[:, :-1].contiguous(), win[:, 1:].contiguous()
    hp = llmt.hparams()
    ctx.set_graph(graph)
    step = 1
    for _ in range(warmup):
        ctx.step(tok, tgt, hp, step)
        step += 1
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    losses = []
    for _ in range(steps):
        losses.append(ctx.step(tok, tgt, hp, step))
        step += 1
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    print(f"bench: {cfg} timed {steps} steps, {dt / steps * 1e3:.3f} ms/step", file=sys.stderr,
          flush=True)
    kinds = ctx.profile_kernels(tok, tgt, hp, step, reps=5 if cfg == "c2" else 2)
    ctx.close()
    if kinds_md:
        print(kinds_markdown(cfg, kinds), flush=True)
    roofline = roofline_obj(cfg, kinds, None, "frozen-weight GEMMs of the step")
    roofline["traffic"] = measured_traffic(f"gemm_{cfg}_traffic")
    # the metric's "bwd % MFMA / HBM peak": the backward's dX GEMMs alone
    roofline_bwd = roofline_obj(cfg, kinds, is_backward_gemm,
                                "backward dX GEMMs (layers and lm_head)")
    roofline_bwd["traffic"] = measured_traffic(f"gemm_{cfg}_traffic", "bwd_traffic_bytes_per_launch")
    bw = bandwidth_kernels(kinds)
    for name, obj in bw.items():
        obj["traffic"] = measured_traffic(f"bandwidth_{cfg}_traffic", f"{name}_traffic_bytes")
    ms = dt / steps * 1e3
    return {
        "value": round(T * steps / dt, 2), "ms_per_step": round(ms, 4), "steps": steps,
        "warmup": warmup, "T": T, "batch": batch, "seq_len": seq_len, "workload": workload,
        "roofline": roofline, "roofline_bwd": roofline_bwd, "kernels": kernel_summary(kinds),
        "kernels_sum_ms": round(sum(k["us"] * k["launches"] for k in kinds) / 1e3, 4),
        "launches_per_step": sum(k["launches"] for k in kinds),
        "bandwidth_kernels": bw,
        "loss_first_last": [round(losses[0], 5), round(losses[-1], 5)],
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", choices=["c1", "c2", "c3", "c4"], default="c2")
    ap.add_argument("--only", action="store_true",
                    help="the selected config alone (no c3 / c4 sub-objects in the c2 line)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--copy-cal", action="store_true", help="PMC byte-counter calibration")
    ap.add_argument("--kinds-md", action="store_true",
                    help="also print the per-kind markdown table of the step (before the line)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py: this build runs on one GPU only (asked for {a.gpus}); the multi-GPU "
              "sharding is a design note, not a code path.", file=sys.stderr)
        sys.exit(2)
    if a.copy_cal:
        copy_calibration()
        return
    if a.config in ("c3", "c1"):
        r = (bench_c3 if a.config == "c3" else bench_c1)(a.steps, a.warmup)
        if not a.no_cpu:
            r["cpu_baseline"] = (cpu_baseline_c3 if a.config == "c3" else cpu_baseline_c1)()
        print(json.dumps(r), flush=True)
        return

    r = bench_step(a.config, a.steps, a.warmup, graph=not a.no_graph, kinds_md=a.kinds_md)
    out = {
        "metric": METRIC,
        "value": r["value"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": r["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (random N(0,0.02) frozen weights, uniform token ids)",
        "config": {"workload": r["workload"], "global_batch": r["batch"], "seq_len": r["seq_len"],
                   "tokens_per_step": r["T"], "graph": not a.no_graph},
        "roofline": r["roofline"],
        "roofline_bwd": r["roofline_bwd"],
        "kernels": r["kernels"],
        "kernels_sum_ms": r["kernels_sum_ms"],
        "launches_per_step": r["launches_per_step"],
        "bandwidth_kernels": r["bandwidth_kernels"],
        "loss_first_last": r["loss_first_last"],
    }
    if a.config == "c2" and not a.only:
        # the other headline configurations, measured in the same run
        c4 = bench_step("c4", min(a.steps, 10), 2, graph=not a.no_graph,
                        kinds_md=a.kinds_md)
        out["c4"] = {k: c4[k] for k in ("workload", "value", "ms_per_step", "steps", "warmup",
                                        "roofline", "roofline_bwd", "kernels", "kernels_sum_ms",
                                        "launches_per_step", "bandwidth_kernels",
                                        "loss_first_last")}
        out["c4"]["unit"] = "tokens/s"
        out["c3"] = bench_c3(min(a.steps, 20), 3)
        out["c1"] = bench_c1(min(a.steps, 20), 3)
    out["achievable"] = achievable_peaks()
    # the C4 GEMM family beside hipBLASLt's fp16 GEMM rate measured in this run
    if "c4" in out:
        blas = out["achievable"]["mfma_f16_tflops_hipblaslt"]
        for key in ("roofline", "roofline_bwd"):
            out["c4"][key]["hipblaslt_tflops"] = blas
            out["c4"][key]["frac_of_hipblaslt"] = round(out["c4"][key]["achieved"] / blas, 4)
    # each bandwidth kernel beside the device copy rate measured in this run
    copy_gbs = out["achievable"]["hbm_copy_gbs"]
    for obj in (out, out.get("c4", {})):
        for k in obj.get("bandwidth_kernels", {}).values():
            k["copy_gbs"] = copy_gbs
            k["copy_frac"] = round(k["gbs"] / copy_gbs, 4)
    if not a.no_cpu:
        if a.config == "c2":
            out["cpu_baseline"] = cpu_baseline(r["batch"], r["seq_len"])
            if "c4" in out:
                out["c4"]["cpu_baseline"] = cpu_baseline_sampled(8, 512)
            if "c3" in out:
                out["c3"]["cpu_baseline"] = cpu_baseline_c3()
            if "c1" in out:
                out["c1"]["cpu_baseline"] = cpu_baseline_c1()
        else:
            out["cpu_baseline"] = cpu_baseline_sampled(r["batch"], r["seq_len"])
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
