"""Benchmark: fused attention forward + backward on one MI355X.

Workload (the headline config): n_embed=1280,
n_head=10, n_kv_head=5, head_dim=128, T=2048, B=16, bf16 fast mode, full
causal window, RMS-normalised Q/K, V ~ N(0,1), dO ~ N(0,0.1), synthetic data.
A step is one forward (O, l, m) plus one backward (dQ, dK, dV, overwrite)
over the whole batch, with every input resident in HBM.

value = algorithmic TFLOP/s = 14 * D * visible_pairs / step time (the
FlashAttention convention: fwd 4*D, bwd 10*D per visible (q,k) pair).
The per-kernel durations come from HIP events the library records around
each of its launches on the launch stream during the timed steps.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, published
PEAK_FP32_TFLOPS = 157.3   # MI355X dense fp32 MFMA, published
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E, published

METRIC = "attention fwd+bwd TFLOP/s and % MFMA peak on 1 MI355X; vs Julia CPU ref"


def kernel_flops(name: str, D: int, pairs: int, B: int, T: int, H: int) -> tuple:
    """(bound, algorithmic amount per launch, unit) of one library kernel.

    fwd: the two products S=QK^T and O=PV, 4*D per visible pair.
    dkdv: the four products S, dP, dV, dK, 8*D per pair.
    dq: the dQ product only, 2*D per pair (its S/dP recomputation is overhead).
    pre: HBM bytes: read dO, O (bf16), l, m; write Delta, lse2 (fp32).
    """
    if name.startswith("attn_fwd"):
        return "mfma", 4 * D * pairs, "flop"
    if name.startswith("attn_bwd_dkdv"):
        return "mfma", 8 * D * pairs, "flop"
    if name.startswith("attn_bwd_dq"):
        return "mfma", 2 * D * pairs, "flop"
    if name.startswith("attn_bwd_pre"):
        return "hbm", B * T * H * (2 * D * 2 + 4 * 4), "byte"
    return "hbm", 0, "byte"


def measured_traffic(workload: str) -> dict:
    """HBM bytes per launch by kernel, from rocprofv3 FETCH_SIZE/WRITE_SIZE runs
    (scaled by a copy-kernel calibration) committed in profiles/."""
    path = os.path.join(ROOT, "profiles", f"attn_{workload.lower()}_hbm_traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
    except OSError:
        return {}
    if data.get("workload") != workload:
        return {}
    return {k: v["read_bytes"] + v["write_bytes"] for k, v in data.get("kernels", {}).items()}


def cpu_baseline(wl, rows: int, threads: int) -> dict:
    """Time the reference's blocked CPU attention (oracle/fa1_blas.py: the
    loop nest and 512-wide blocks of flash_attention₁!/Δflash_attention₁!,
    src/kernels.jl:131-379, no block skipping, every product a BLAS sgemm as
    the reference's mul! calls) on a bounded sample of the same workload:
    ``rows`` batch rows, all heads, bf16-rounded inputs in float32 (the
    reference's CPU path computes in the input type; its BFloat16 matmul is a
    generic fallback, so the fp32 path is the one to time)."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from femtochat_amd import workloads as W
    from oracle import fa1_blas

    h = W.host_inputs(wl, 0, batch=list(range(rows)))
    with threadpool_limits(limits=threads, user_api="blas"):
        blas = fa1_blas.blas_info()
        fa1_blas.forward(h.Q[:1, :512], h.K[:1, :512], h.V[:1, :512], h.window)  # warm-up (pages, threads)
        t0 = time.perf_counter()
        O, l, m = fa1_blas.forward(h.Q, h.K, h.V, h.window, h.positions)
        t1 = time.perf_counter()
        fa1_blas.backward(h.dO, h.Q, h.K, h.V, O, l, m, h.window, h.positions)
        t2 = time.perf_counter()
    pairs = W.visible_pairs(wl.T, rows, wl.H, h.window, h.positions)
    flop = 14 * wl.D * pairs
    assert np.isfinite(O).all()
    return {
        "value": flop / (t2 - t0) / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "blas": blas,
        "fwd_s": round(t1 - t0, 3),
        "bwd_s": round(t2 - t1, 3),
        "sample": (f"{wl.name} batch rows 0..{rows - 1} of {wl.B}, all {wl.H} heads, T={wl.T}: fwd {t1 - t0:.2f} s "
                   f"+ bwd {t2 - t1:.2f} s; the reference's blocked algorithm (flash_attention₁!/Δflash_attention₁!, "
                   "src/kernels.jl:131-379: 512-blocks, no skipping, products as BLAS sgemm) in float32 on "
                   f"bf16-rounded inputs, {blas.get('library', 'BLAS')} {blas.get('version', '')} with "
                   f"{blas.get('threads', threads)} threads (the Python loop itself single-threaded, as the "
                   "reference's Julia loop); TFLOP/s counts algorithmic visible-pair FLOPs like the GPU value"),
    }


def measure_prologue(wl, dev, steps: int) -> dict:
    """The attention prologue (rotary embedding + RMS norm x 1.2) on the
    workload's Q and K, forward and backward (overwrite), bf16: HBM-bound, so
    its roofline is algorithmic bytes (X read, Y written; dY and X read, dX
    written) per unit time against 8 TB/s.  Not part of the headline value."""
    import torch

    import femtochat_amd._lib as L
    from femtochat_amd import attention_prologue_, delta_attention_prologue_, rotary_embeddings

    sin, cos = rotary_embeddings(wl.T, wl.D, device=dev)
    g = torch.Generator(device=dev).manual_seed(0)
    Xs = [torch.randn(wl.B, wl.T, nh, wl.D, device=dev, generator=g).to(torch.bfloat16) for nh in (wl.H, wl.Hkv)]
    Ys = [torch.empty_like(x) for x in Xs]
    dXs = [torch.empty_like(x) for x in Xs]

    def once():
        for X, Y in zip(Xs, Ys):
            attention_prologue_(Y, X, (sin, cos))
        for X, Y, dX in zip(Xs, Ys, dXs):
            delta_attention_prologue_(dX, Y, X, (sin, cos), accumulate=False)

    for _ in range(3):
        once()
    torch.cuda.synchronize()
    L.profile_collect()
    L.profile_enable(True)
    for _ in range(steps):
        once()
    torch.cuda.synchronize()
    L.profile_enable(False)
    k = L.profile_collect()
    nbytes = sum(x.numel() * x.element_size() for x in Xs)
    out = {"workload": f"{wl.name} Q (B,T,H,D) and K (B,T,Hkv,D), bf16, no positions"}
    traffic = measured_traffic(wl.name)
    for name, mult in (("rope_norm_fwd_bf16", 2), ("rope_norm_bwd_bf16", 3)):
        n, tot = k[name]
        per_step_ms = tot / steps  # both tensors
        achieved = mult * nbytes / (per_step_ms * 1e-3) / 1e9
        key = "fwd" if "fwd" in name else "bwd"
        out[key] = {"ms_per_step": round(per_step_ms, 4), "launches": n,
                    "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                                 "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                                 # rocprof's bytes per launch (averaged over the Q and K launches) x 2
                                 "traffic": (2 * traffic[name.replace("_bf16", "")]
                                             if name.replace("_bf16", "") in traffic else None)}}
    return out


def measure_loss(dev, steps: int) -> dict:
    """Loss-side kernels at the training step's shape (scripts/train.jl
    defaults: vocabulary 2^15, 4 x 2048 tokens, 512-wide embeddings; fp32
    logits and weights): cross-entropy forward (losses, log-sum-exp, mean),
    its gradient accumulating into the logits' gradient, both in one pass
    (fused, writing the gradient), the embedding gather
    and its scatter-add gradient.  HBM-bound: algorithmic bytes per unit time
    against 8 TB/s.  Not part of the headline value."""
    import torch

    import femtochat_amd._lib as L
    from femtochat_amd import (cross_entropy_, cross_entropy_fused_, cross_entropy_gradient_, embedding_,
                               embedding_gradient_)

    V, N, D = 32768, 4 * 2048, 512
    g = torch.Generator(device=dev).manual_seed(0)
    logits = torch.randn(N, V, device=dev, generator=g) * 4
    targets = torch.randint(0, V, (N,), device=dev, generator=g, dtype=torch.int32)
    dlogits = torch.zeros_like(logits)
    losses, lse = torch.empty(N, device=dev), torch.empty(N, device=dev)
    reduced, count = torch.empty(1, device=dev), torch.empty(1, device=dev)
    dy = torch.ones(1, device=dev)
    W = torch.randn(V, D, device=dev, generator=g)
    dW = torch.zeros_like(W)
    tokens = torch.randint(0, V, (N,), device=dev, generator=g, dtype=torch.int32)
    y = torch.empty(N, D, device=dev)
    dY = torch.randn(N, D, device=dev, generator=g)

    def once():
        cross_entropy_(losses, logits, targets, -1, "mean", lse=lse, reduced=reduced, count=count)
        cross_entropy_gradient_(dlogits, logits, targets, dy, -1, "mean", lse=lse, count=count)
        cross_entropy_fused_(losses, dlogits, logits, targets, dy, -1, "mean", lse=lse, count=count)
        embedding_(y, W, tokens)
        embedding_gradient_(dW, dY, tokens)

    for _ in range(3):
        once()
    torch.cuda.synchronize()
    L.profile_collect()
    L.profile_enable(True)
    for _ in range(steps):
        once()
    torch.cuda.synchronize()
    L.profile_enable(False)
    k = L.profile_collect()
    lg, em = N * V * 4, N * D * 4
    out = {"workload": f"train.jl step: V={V}, N={N} tokens (B=4, T=2048), D={D}, fp32; uniform random targets/tokens"}
    # bytes per launch: logits read; logits read + gradient read and written;
    # fused: logits read + gradient written; weight rows read + output written;
    # dy read + weight rows read and written
    for name, nbytes in (("xent_fwd", lg), ("xent_bwd", 3 * lg), ("xent_fused", 2 * lg), ("embed_fwd", 2 * em),
                         ("embed_bwd", 3 * em)):
        n, tot = k[name]
        ms = tot / steps
        achieved = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"ms": round(ms, 4), "launches": n, "bytes": nbytes,
                     "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                                  "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4)}}
    # the deterministic gradient (key kernel, radix sort passes, one in-order
    # sum per id), timed with events around the whole call
    from femtochat_amd.loss import embedding_gradient_workspace_bytes
    ws = torch.empty(embedding_gradient_workspace_bytes(dW, tokens), dtype=torch.uint8, device=dev)
    for _ in range(3):
        embedding_gradient_(dW, dY, tokens, deterministic=True, workspace=ws)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        embedding_gradient_(dW, dY, tokens, deterministic=True, workspace=ws)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    achieved = 3 * em / (ms * 1e-3) / 1e9
    out["embed_bwd_sorted"] = {"ms": round(ms, 4), "bytes": 3 * em, "deterministic": True,
                               "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                                            "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4)}}
    return out


def measure_optim(dev, steps: int) -> dict:
    """Optimizer kernels at the training model's sizes (scripts/train.jl
    defaults: n_embed 512, 8 layers, vocabulary 2^15): one AdamW step over
    2^26 fp32 parameters (the embedding, value-embedding and head matrices'
    scale), Muon's final write over the block matrices, and Polar Express
    (5 steps, fp32 and bf16) over their stacks: 32 of 512x512, 8 of 512x2048
    and 8 of 2048x512.  AdamW and the write are HBM-bound (bytes per unit time
    against 8 TB/s); Polar Express is batched products (rocBLAS in fp32, the
    library's MFMA kernel in bf16): FLOP per unit time against the fp32 or
    bf16 MFMA peak.  Not part of the headline value."""
    import torch

    from femtochat_amd import AdamW, muon_update_, polar_express_
    from femtochat_amd.optim import polar_express_grouped_, polar_workspace_bytes

    g = torch.Generator(device=dev).manual_seed(0)
    n = 1 << 26
    theta = torch.randn(n, device=dev, generator=g)
    grad = torch.randn(n, device=dev, generator=g)
    opt = AdamW(theta, alpha=0.004, beta1=0.8, beta2=0.96, eps=1e-10, lam=0.01)
    shapes = [(512, 512, 32), (512, 2048, 8), (2048, 512, 8)]  # Julia (m, n, k)
    stacks = [torch.randn(k, nn, mm, device=dev, generator=g) for mm, nn, k in shapes]
    work = [torch.empty(polar_workspace_bytes(G), dtype=torch.uint8, device=dev) for G in stacks]
    flat_n = sum(G.numel() for G in stacks)
    Theta = torch.randn(flat_n, device=dev, generator=g)
    offs, pos = [], 0
    for G in stacks:
        w = G[0].numel()
        offs.append(torch.arange(G.shape[0], device=dev, dtype=torch.int64) * w + pos)
        pos += G.numel()
    eta, lam = torch.tensor([0.02], device=dev), torch.tensor([0.01], device=dev)

    def timed(fn, reps):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    out = {"workload": "train.jl model: AdamW over 2^26 fp32 parameters; Muon stacks 32x(512x512), "
                       "8x(512x2048), 8x(2048x512), fp32, 5 Polar Express steps"}
    ms = timed(lambda: opt(theta, grad), steps)
    nbytes = 28 * n  # theta, grad, m, v read; theta, m, v written
    out["adamw"] = {"ms": round(ms, 4), "bytes": nbytes, "roofline": _hbm_roofline(nbytes, ms)}
    for G, o in zip(stacks, offs):  # offsets checked once, outside the timed region
        muon_update_(Theta, G.reshape(G.shape[0], -1), eta, lam, o)
    ms = timed(lambda: [muon_update_(Theta, G.reshape(G.shape[0], -1), eta, lam, o, validate=False)
                        for G, o in zip(stacks, offs)], steps)
    nbytes = 12 * flat_n  # Theta read and written, X read
    out["muon_update"] = {"ms": round(ms, 4), "bytes": nbytes, "roofline": _hbm_roofline(nbytes, ms)}
    flops = 0
    for mm, nn, k in shapes:
        lo, hi = min(mm, nn), max(mm, nn)
        flops += 5 * k * (4 * lo * lo * hi + 2 * lo ** 3)
    ms = timed(lambda: [polar_express_(G, 5, w) for G, w in zip(stacks, work)], max(2, steps // 4))
    achieved = flops / (ms * 1e-3) / 1e12
    out["polar_express"] = {"ms": round(ms, 4), "flop": flops, "compute": "fp32",
                            "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP32_TFLOPS,
                                         "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_TFLOPS, 4)}}
    # scripts/train.jl passes compute_type=BFloat16 to MuonAdamW: the iteration in bf16
    work16 = [torch.empty(polar_workspace_bytes(G, 5, torch.bfloat16), dtype=torch.uint8, device=dev) for G in stacks]
    ms = timed(lambda: [polar_express_(G, 5, w, compute_type=torch.bfloat16) for G, w in zip(stacks, work16)],
               max(2, steps // 4))
    achieved = flops / (ms * 1e-3) / 1e12
    out["polar_express_bf16"] = {"ms": round(ms, 4), "flop": flops, "compute": "bf16 (fp32 accumulation)",
                                 "roofline": {"bound": "mfma", "achieved": round(achieved, 2),
                                              "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                                              "frac": round(achieved / PEAK_BF16_TFLOPS, 4)}}
    # the three stacks in one grouped call (concurrent on helper streams)
    ms = timed(lambda: polar_express_grouped_(stacks, 5, work16, compute_type=torch.bfloat16), max(2, steps // 4))
    achieved = flops / (ms * 1e-3) / 1e12
    out["polar_express_bf16_grouped"] = {"ms": round(ms, 4), "flop": flops, "compute": "bf16, stacks concurrent",
                                         "roofline": {"bound": "mfma", "achieved": round(achieved, 2),
                                                      "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                                                      "frac": round(achieved / PEAK_BF16_TFLOPS, 4)}}
    return out


def _hbm_roofline(nbytes: int, ms: float) -> dict:
    achieved = nbytes / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4)}


def measure_attention(wl, dev, steps: int, warmup: int, accumulate: bool = False) -> dict:
    """One fwd+bwd step (every layer of the workload; gradients overwritten,
    or added to the buffers' values with ``accumulate``) timed over
    ``steps`` after ``warmup``, with per-kernel times from the library's HIP
    events on the launch stream."""
    import torch

    import femtochat_amd._lib as L
    from femtochat_amd import (MFMAExact, MFMAFast, attention_, backward_workspace_bytes, delta_attention_,
                               forward_workspace_bytes)
    from femtochat_amd import workloads as W

    fast = wl.mode == "fast"
    A = MFMAFast() if fast else MFMAExact()
    layers = []
    total_pairs = 0
    for layer in range(wl.layers):
        Q, K, V, dO, pos, window = W.device_inputs(wl, layer, dev)
        O = torch.empty_like(Q)
        l = torch.empty((wl.B, wl.H, wl.T), device=dev)
        m = torch.empty((wl.B, wl.H, wl.T), device=dev)
        dQ, dK, dV = torch.zeros_like(Q), torch.zeros_like(K), torch.zeros_like(V)
        ws = torch.empty(backward_workspace_bytes(A, Q, K, positions=pos), dtype=torch.uint8, device=dev)
        nf = forward_workspace_bytes(A, Q, K, positions=pos)
        fws = torch.empty(nf, dtype=torch.uint8, device=dev) if nf > 0 else None
        pairs = W.visible_pairs(wl.T, wl.B, wl.H, window, None if pos is None else pos.cpu().numpy())
        total_pairs += pairs
        layers.append((Q, K, V, dO, pos, window, O, l, m, dQ, dK, dV, ws, fws))

    def step():
        for (Q, K, V, dO, pos, window, O, l, m, dQ, dK, dV, ws, fws) in layers:
            attention_(A, O, l, m, Q, K, V, window, positions=pos, workspace=fws)
            delta_attention_(A, dQ, dK, dV, dO, Q, K, V, O, l, m, window, positions=pos, accumulate=accumulate,
                             workspace=ws)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    L.profile_collect()  # discard anything recorded before
    L.profile_enable(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    L.profile_enable(False)
    kernels = L.profile_collect()

    ms = (t1 - t0) * 1e3 / steps
    flop = 14 * wl.D * total_pairs
    value = flop / (ms * 1e-3) / 1e12
    peak = PEAK_BF16_TFLOPS if fast else PEAK_FP32_TFLOPS
    per_kernel = {}
    for name, (n, tot) in sorted(kernels.items()):
        avg = tot / n
        bound, amount, unit = kernel_flops(name, wl.D, total_pairs // wl.layers, wl.B, wl.T, wl.H)
        rate = amount / (avg * 1e-3)
        kpeak = peak if bound == "mfma" else PEAK_HBM_GBS
        achieved = rate / (1e12 if unit == "flop" else 1e9)
        per_kernel[name] = {"launches": n, "avg_ms": round(avg, 4), "bound": bound, "achieved": round(achieved, 2),
                            "unit": "TFLOP/s" if unit == "flop" else "GB/s", "frac": round(achieved / kpeak, 4)}
    del layers
    torch.cuda.empty_cache()
    return {"workload": f"{wl.name}: {wl.description}", "mode": wl.mode, "layers": wl.layers,
            "ms_per_step": round(ms, 4), "tflops": round(value, 2), "peak_tflops": peak,
            "peak_frac": round(value / peak, 4), "visible_pairs": total_pairs, "flop_per_step": flop,
            "steps": steps, "kernels": per_kernel, "raw": kernels}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="C3")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-rows", type=int, default=16, help="batch rows in the CPU baseline sample")
    ap.add_argument("--configs", default="C1,C2,C4,C5",
                    help="other BASELINE workloads timed beside the headline (comma list; '' for none)")
    ap.add_argument("--sections", default="accumulate,prologue,loss,optim",
                    help="measurements besides the headline attention step (comma list of accumulate, prologue, "
                         "loss, optim; 'none' for only the headline)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every box in this build has a single MI355X, and the attention "
              f"kernels need no collective (--gpus {args.gpus} is not supported).", file=sys.stderr)
        return 2

    import torch

    from femtochat_amd import workloads as W

    wl = W.WORKLOADS[args.workload]
    dev = torch.device("cuda", 0)
    fast = wl.mode == "fast"
    head = measure_attention(wl, dev, args.steps, args.warmup)
    ms, flop, value, peak = head["ms_per_step"], head["flop_per_step"], head["tflops"], head["peak_tflops"]
    total_pairs, per_kernel, kernels = head["visible_pairs"], head["kernels"], head["raw"]
    dominant = max(kernels.items(), key=lambda kv: kv[1][1])[0]
    dk = per_kernel[dominant]
    dpeak = peak if dk["bound"] == "mfma" else PEAK_HBM_GBS
    traffic = measured_traffic(wl.name)
    dom_key = next((k for k in traffic if dominant.startswith(k)), None)
    roofline = {"kernel": dominant, "bound": dk["bound"], "achieved": dk["achieved"], "peak": dpeak,
                "unit": dk["unit"], "frac": round(dk["achieved"] / dpeak, 4),
                "traffic": traffic[dom_key] if dom_key else None}
    for name, rec in per_kernel.items():
        key = next((k for k in traffic if name.startswith(k)), None)
        if key:
            rec["hbm_bytes"] = traffic[key]
            rec["hbm_gbs"] = round(traffic[key] / (rec["avg_ms"] * 1e-3) / 1e9, 1)

    # The other BASELINE configurations, each a full step (all its layers):
    # parity cases in tests/, timed here beside the headline.
    configs = {}
    for name in [c for c in args.configs.split(",") if c and c != wl.name]:
        r = measure_attention(W.WORKLOADS[name], dev, max(3, args.steps), max(2, args.warmup))
        r.pop("raw")
        configs[name] = r

    # The headline workload once more with the reference's default backward
    # semantics (gradients added to the buffers' values, src/kernels.jl:420).
    requested = set(args.sections.split(","))
    accumulated = None
    if "accumulate" in requested:
        acc = measure_attention(wl, dev, args.steps, args.warmup, accumulate=True)
        accumulated = {"ms_per_step": acc["ms_per_step"], "tflops": acc["tflops"], "peak_frac": acc["peak_frac"],
                       "kernels": {k: v["avg_ms"] for k, v in acc["kernels"].items()}}

    sections = requested if fast else set()
    prologue = measure_prologue(wl, dev, args.steps) if "prologue" in sections else None
    loss_side = measure_loss(dev, args.steps) if "loss" in sections else None
    optim_side = measure_optim(dev, args.steps) if "optim" in sections else None

    cpu = None
    if not args.no_cpu:
        threads = min(16, os.cpu_count() or 1)
        cpu = cpu_baseline(wl, min(args.cpu_rows, wl.B), threads)
        cpu["value"] = round(cpu["value"], 5)

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if fast else "f32",
        "data": "synthetic",
        "config": {
            "workload": f"{wl.name}: {wl.description}",
            "D": wl.D, "H": wl.H, "Hkv": wl.Hkv, "T": wl.T, "B": wl.B, "windows": [list(w) for w in wl.windows],
            "mode": wl.mode, "visible_pairs": total_pairs, "flop_per_step": flop,
            "mfma_peak_frac": round(value / peak, 4), "peak_tflops": peak,
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": per_kernel,
        "configs": configs,
        "accumulate": accumulated,
        "prologue": prologue,
        "loss": loss_side,
        "optim": optim_side,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
