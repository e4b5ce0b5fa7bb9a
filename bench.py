"""Benchmark: MoE-layer forward + backward tokens/s on one MI355X.

Workload: the Mixtral-shaped layer (T = 2 x 2048 tokens, d_model 4096, 8 experts,
top-2 sigmoid router, SwiGLU hidden 14336, bf16 with fp32 accumulation), built by
the workload recipe on the host (seeded module init, N(0, 0.02^2) weights, N(0, 1)
activations and target), then moved to the GPU.  One step = forward of the layer,
MSE loss against the target, backward to x and every parameter (train mode, so the
router's bias step runs too; the bias is reset before every step, so every step
routes the same way).  Forward-only workloads (the small skewed batches) run the
forward under no_grad.

Prints one JSON line with the throughput, the roofline position of the dominant
kernel (device time from HIP events recorded on the launch stream around every
entry point during the timed steps), per-kernel figures, and the CPU baseline: the
oracle's restatement of the reference algorithm timed on the host cores on a bounded
token sample of the same layer.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

import torch

# MI355X published peaks
PEAK_BF16_TFLOPS = 2500.0
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0

METRIC = "MoE-layer fwd+bwd tokens/sec on 1 MI355X; grouped-GEMM MFMA util %, dispatch GB/s"

GEMM_FLOPS = {  # multiples of R*D*M per entry point
    "abacus_moe_gateup_fwd": 4,
    "abacus_moe_down_fwd": 2,
    "abacus_moe_down_bwd_dgrad": 2,
    "abacus_moe_down_bwd_wgrad": 2,
    "abacus_moe_down_bwd": 4,            # dgrad + wgrad in one launch
    "abacus_moe_gateup_bwd_dgrad": 4,
    "abacus_moe_gateup_bwd_wgrad": 4,
    "abacus_moe_gateup_bwd": 8,          # dgrad + wgrad in one launch
}


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--workload", default="mixtral_bf16",
                   help="an MoE-layer workload of abacus_amd.workloads, or decoder_bf16 / decoder_fp32 "
                        "(the full MoE decoder training step)")
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="target CPU-baseline sample duration")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-graph", action="store_true", help="skip the HIP-graph replay of forward-only workloads")
    p.add_argument("--vendor-gemm", action="store_true",
                   help="instead of the layer step: time hipBLASLt (torch.mm) on the same per-expert products "
                        "as the four grouped-GEMM entry points, with the workload's own routing (a reference "
                        "point for the GEMM kernels; no fused epilogues)")
    p.add_argument("--gemm-shapes", action="store_true",
                   help="instead of the layer step: time the four grouped-GEMM entry points with the workload's "
                        "rows split as its routing splits them, as E equal experts and as one expert (a dense "
                        "product), beside hipBLASLt on the dense product of the same size")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="after the timed steps, copy 1 GiB device-to-device once (a known-size kernel "
                        "to scale FETCH_SIZE / WRITE_SIZE counters against)")
    return p.parse_args()


def hbm_bytes(wl, name):
    """Algorithmic HBM bytes per launch for the memory-bound entry points."""
    s, T, R, D, K = wl.elem_bytes(), wl.tokens, wl.rows, wl.dim, wl.top_k
    if name in ("abacus_moe_permute_gather", "abacus_moe_dispatch"):
        return wl.dispatch_bytes()
    if name == "abacus_moe_combine_fwd":
        return wl.combine_bytes()
    if name == "abacus_moe_combine_bwd":
        # read dout once and every routed y row, write every routed dy row; weights/scores/rows/dlogit
        return s * D * (T + 2 * R) + (s + 4 + 4 + 4) * R
    if name == "abacus_moe_unpermute_bwd":
        return s * D * (R + T) + (4 + 4 + 4) * R
    E = wl.n_experts
    if name == "abacus_moe_router_fwd":
        # read x and w_DE; write logits, weights, int64 + int32 indices and fp32 scores
        return s * T * D + s * D * E + s * T * E + (s + 8 + 4 + 4) * T * K
    if name == "abacus_moe_router_wgrad":
        # read x, the fp32 dlogits and int32 indices; write dW_DE
        return s * T * D + (4 + 4) * T * K + s * D * E
    return None


def weight_stream_bytes(wl, e_touched):
    """Bytes per launch of the forward expert products at decode-sized batches (inference: no G, U
    saved): the touched experts' weights, the routed rows in, the product rows out."""
    s, R, D, M = wl.elem_bytes(), wl.rows, wl.dim, wl.hidden
    return {
        "abacus_moe_gateup_fwd": s * (2 * e_touched * D * M + R * D + R * M),
        "abacus_moe_down_fwd": s * (e_touched * M * D + R * M + R * D),
    }


TRAFFIC_FILE = "profiles/hbm_traffic_mixtral_bf16_fwd_bwd.md"


def measured_traffic(name):
    """HBM bytes per launch of an entry point from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), TRAFFIC_FILE)
    try:
        with open(path) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 3 and parts[0] == "traffic" and parts[1] == name:
                    return int(parts[2])
    except OSError:
        pass
    return None


def cpu_baseline(wl, state, x_cpu, target_cpu, target_seconds):
    """Oracle (the reference algorithm restated) on host cores, on the same layer's weights and
    the first tokens of the same inputs (a bounded sample)."""
    from oracle import moe_oracle as oracle

    cores = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(cores)
    D, K = wl.dim, wl.top_k
    w_DE, wg, wu, wd = (state[k] for k in ("router.w_DE", "w_gate_EDM", "w_up_EDM", "w_down_EMD"))
    bias = state["router.expert_bias_E"]
    xs, ts = x_cpu.reshape(-1, D), target_cpu.reshape(-1, D)

    def run(tokens):
        x = xs[:tokens].clone().requires_grad_(wl.backward)
        params = [t.clone().requires_grad_(wl.backward) for t in (w_DE, wg, wu, wd)]
        t0 = time.perf_counter()
        with torch.set_grad_enabled(wl.backward):
            out, _ = oracle.moe_forward(x, params[0], bias, params[1], params[2], params[3], K, 1.0)
            if wl.backward:
                loss = (out.float() - ts[:tokens].float()).pow(2).mean()
                loss.backward()
        return time.perf_counter() - t0

    # Sample size: a step of the reference algorithm costs a fixed part (its per-expert weight
    # slices and their gradients, once every expert has tokens) plus a part per token, fitted from
    # n1 = 256 and n2 = 1024 tokens (16 and T for smaller batches; below a few hundred tokens the
    # number of active experts still grows, which a fit from 16 tokens reads as per-token cost).
    # The sample is the most tokens whose predicted step fits a third of the time budget, raised
    # (up to a 30 s step) until the per-token part is at least three quarters of the step, so the
    # rate measures the per-token work the GPU is compared on rather than the fixed part.
    run(16)  # warm-up
    n1, n2 = (256, min(1024, wl.tokens)) if wl.tokens > 256 else (16, wl.tokens)
    t1, t2 = run(n1), run(n2)
    per_token = max((t2 - t1) / max(n2 - n1, 1), 1e-7)
    fixed = max(t1 - n1 * per_token, 0.0)
    budget_tokens = (target_seconds / 3 - fixed) / per_token
    dominant_tokens = min(3 * fixed / per_token, (30.0 - fixed) / per_token)
    tokens = int(min(wl.tokens, max(16, budget_tokens, dominant_tokens)))
    times = [run(tokens)]
    while sum(times) < target_seconds and len(times) < 5:
        times.append(run(tokens))
    med = statistics.median(times)
    if tokens > n2:
        # refit on the sample's own step: over n1 .. n2 the fixed part can hide most of the
        # per-token part (the Mixtral shape's 2.8 GB of weights and their gradients)
        per_token = max((med - t1) / (tokens - n1), 1e-7)
        fixed = max(t1 - n1 * per_token, 0.0)
    share = tokens * per_token / (fixed + tokens * per_token)
    full_step = fixed + wl.tokens * per_token
    cpu_model = platform.processor() or "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": tokens / med,
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "fit": {"fixed_s_per_step": round(fixed, 4), "us_per_token": round(per_token * 1e6, 2),
                "sample_tokens": tokens, "per_token_share_of_sample_step": round(share, 3),
                "predicted_full_step_s": round(full_step, 3),
                "predicted_full_step_tokens_per_s": round(wl.tokens / full_step, 1)},
        "sample": (f"{wl.name} layer (D={D}, E={wl.n_experts}, K={K}, M={wl.hidden}, "
                   f"{str(wl.dtype).replace('torch.', '')}, the benchmark's own weights) on the first {tokens} of its "
                   f"{wl.tokens} tokens, {'fwd+bwd' if wl.backward else 'fwd'} of the oracle's restatement of "
                   f"router.py:40-70 + moe.py:60-86, median of {len(times)} runs ({med:.2f} s each; fitted fixed "
                   f"cost per step {fixed:.2f} s + {per_token * 1e6:.1f} us per token, the per-token part "
                   f"{100 * share:.0f}% of the sample's step); torch CPU threads={cores}, "
                   f"os.cpu_count={os.cpu_count()}, cpu='{cpu_model}'"),
    }


# The full small MoE decoder training step (transformer_moe.py architecture):
# 8 layers, d_model 1024, 16 heads of 64 with RoPE and QK-norm, vocab 32000, an
# MoE FFN in every layer (16 experts, top-2, SwiGLU hidden 2816); batch 4 x
# 2048 token ids uniform in [0, 32000), seed 4; one AdamW step per step.
DECODER = dict(dim=1024, n_heads=16, head_dim=64, n_blocks=8, vocab_size=32000, n_experts=16, top_k=2,
               hidden_dim=2816)
DECODER_BATCH, DECODER_SEQ, DECODER_SEED = 4, 2048, 4


def bench_decoder(args, dtype):
    """Training-step tokens/s of the MoE decoder and the MoE kernels' share of the step."""
    from abacus_amd import _lib
    from abacus_amd.train import make_optimizer, train_step
    from abacus_amd.transformer import TransformerMoe

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    torch.manual_seed(DECODER_SEED)
    model = TransformerMoe(**DECODER)  # built on the host: the reference constructors' RNG order
    tokens = torch.randint(0, DECODER["vocab_size"], (DECODER_BATCH, DECODER_SEQ))
    model = model.to(dtype).to(dev)
    tokens = tokens.to(dev)
    opt = make_optimizer(model)
    for _ in range(args.warmup):
        train_step(model, opt, tokens)
    torch.cuda.synchronize()
    losses = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        losses.append(train_step(model, opt, tokens))
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = 1000.0 * elapsed / args.steps
    # After the timed region: as many steps again with HIP events around every entry point (each
    # event record delays the next kernel by a few microseconds, so none are in the timed steps).
    timer = _lib.KernelTimer()
    t1 = time.perf_counter()
    with timer:
        for _ in range(args.steps):
            train_step(model, opt, tokens)
        torch.cuda.synchronize()
    full_elapsed = time.perf_counter() - t1
    totals = timer.totals_ms()
    moe_ms = sum(ms for name, (ms, _) in totals.items() if name.startswith("abacus_moe_")) / args.steps
    lib_ms = sum(ms for ms, _ in totals.values()) / args.steps  # every entry point: MoE, norms, AdamW
    kernels = {name: {"avg_us": round(ms / n * 1000.0, 2), "calls": n,
                      "share": round(ms / (full_elapsed * 1000.0), 4)}
               for name, (ms, n) in sorted(totals.items(), key=lambda kv: -kv[1][0])}
    tok = DECODER_BATCH * DECODER_SEQ
    n_params = sum(p.numel() for p in model.parameters())
    return {
        "metric": "MoE decoder training step tokens/sec on 1 MI355X (forward, cross-entropy, backward, AdamW)",
        "value": round(tok / (ms_per_step / 1000.0), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if dtype == torch.bfloat16 else "fp32",
        "data": f"synthetic token ids uniform in [0, {DECODER['vocab_size']}), seed {DECODER_SEED}; random init",
        "config": {"workload": f"MoE decoder training step: {DECODER['n_blocks']} layers, d_model {DECODER['dim']}, "
                               f"{DECODER['n_heads']} heads x {DECODER['head_dim']}, vocab {DECODER['vocab_size']}, "
                               f"MoE E={DECODER['n_experts']} K={DECODER['top_k']} M={DECODER['hidden_dim']} in "
                               f"every layer; batch {DECODER_BATCH} x seq {DECODER_SEQ}",
                   "parameters": n_params, "tokens_per_step": tok},
        "moe_share": round(moe_ms / (1000.0 * full_elapsed / args.steps), 4),
        "moe_ms_per_step": round(moe_ms, 4),
        "hip_library_ms_per_step": round(lib_ms, 4),
        "loss_first_last": [round(float(losses[0]), 4), round(float(losses[-1]), 4)],
        "kernels": kernels,
        "timing": {"value": "the timed steps carry no events",
                   "kernels": "HIP events around every entry point over as many further steps",
                   "kernels_pass_ms_per_step": round(1000.0 * full_elapsed / args.steps, 4)},
    }


def bench_vendor_gemm(args, wl, moe, x):
    """hipBLASLt (torch.mm on 2-D operands) on the per-expert products of the four grouped-GEMM
    entry points, expert by expert with the workload's routing: the vendor library's rate on the
    same shapes (operands N(0,1) activations and the module's weights; the library's own kernels
    see no SwiGLU, scaling or fused outputs, so this is a lower bound on their work)."""
    dev = x.device
    moe.eval()
    with torch.no_grad():
        moe(x)
    counts = [int(c) for c in moe.router.last_routing.counts_E.tolist()]
    D, M, dt = wl.dim, wl.hidden, wl.dtype
    g = torch.Generator(device=dev).manual_seed(wl.seed)

    def act(rows, cols):
        return torch.randn(rows, cols, device=dev, generator=g).to(dt)

    xs = [act(s, D) for s in counts]
    hs = [act(s, M) for s in counts]
    dys = [act(s, D) for s in counts]
    dgs = [act(s, M) for s in counts]
    dus = [act(s, M) for s in counts]
    wg, wu, wd = moe.w_gate_EDM.detach(), moe.w_up_EDM.detach(), moe.w_down_EMD.detach()
    out_rm = [torch.empty(s, M, device=dev, dtype=dt) for s in counts]
    out_rd = [torch.empty(s, D, device=dev, dtype=dt) for s in counts]
    out_dm = torch.empty(D, M, device=dev, dtype=dt)
    out_md = torch.empty(M, D, device=dev, dtype=dt)
    experts = [e for e, s in enumerate(counts) if s > 0]

    def gateup_fwd():
        for e in experts:
            torch.mm(xs[e], wg[e], out=out_rm[e])
            torch.mm(xs[e], wu[e], out=out_rm[e])

    def down_fwd():
        for e in experts:
            torch.mm(hs[e], wd[e], out=out_rd[e])

    def down_bwd():
        for e in experts:
            torch.mm(dys[e], wd[e].t(), out=out_rm[e])   # data gradient (before the SwiGLU backward)
            torch.mm(hs[e].t(), dys[e], out=out_md)      # weight gradient

    def gateup_bwd():
        for e in experts:
            torch.mm(dgs[e], wg[e].t(), out=out_rd[e])   # data gradient, gate half
            out_rd[e].addmm_(dus[e], wu[e].t())          # + up half
            torch.mm(xs[e].t(), dgs[e], out=out_dm)      # weight gradients
            torch.mm(xs[e].t(), dus[e], out=out_dm)

    kinds = {"abacus_moe_gateup_fwd": gateup_fwd, "abacus_moe_down_fwd": down_fwd,
             "abacus_moe_down_bwd": down_bwd, "abacus_moe_gateup_bwd": gateup_bwd}
    R = sum(counts)
    res = {}
    for name, fn in kinds.items():
        for _ in range(max(1, args.warmup)):
            fn()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        torch.cuda.synchronize()
        ev[0].record()
        for _ in range(args.steps):
            fn()
        ev[1].record()
        torch.cuda.synchronize()
        us = ev[0].elapsed_time(ev[1]) * 1000.0 / args.steps
        tf = GEMM_FLOPS[name] * R * D * M / (us / 1e6) / 1e12
        res[name] = {"avg_us": round(us, 2), "tflops": round(tf, 1), "mfma_frac": round(tf / PEAK_BF16_TFLOPS, 4)}
    return {"vendor_gemm": "hipBLASLt via torch.mm, per expert, the workload's routing",
            "workload": wl.name, "rows_per_expert": counts, "steps": args.steps, "kinds": res}


def bench_gemm_shapes(args, wl, moe, x):
    """The four grouped-GEMM entry points on the workload's R = T*K rows split three ways -- as
    its routing splits them, as E equal experts, and as one expert (then each kind is a dense
    product) -- and hipBLASLt (torch.mm) on that dense product: what the per-expert structure
    (more weight matrices, ragged row counts) costs each kind, against the vendor library on
    the product without it.  Operands: N(0,1) rows (gradients N(0,1e-4^2)), the module's
    weights (expert 0's for the dense case)."""
    from abacus_amd import _lib

    dev = x.device
    moe.eval()
    with torch.no_grad():
        moe(x)
    counts = [int(c) for c in moe.router.last_routing.counts_E.tolist()]
    D, M, E, dt = wl.dim, wl.hidden, wl.n_experts, wl.dtype
    if dt != torch.bfloat16:
        raise SystemExit("--gemm-shapes times the bf16 kernels")
    R = sum(counts)
    code, s = _lib.dtype_code(dt, dev), _lib.stream_of(dev)
    call, ptr = _lib.call, _lib.ptr
    g = torch.Generator(device=dev).manual_seed(wl.seed)

    def act(rows, cols, scale=1.0):
        return (torch.randn(rows, cols, device=dev, generator=g) * scale).to(dt)

    xp, h = act(R, D), act(R, M)
    dy, dgate, dup = act(R, D, 1e-4), act(R, M, 1e-4), act(R, M, 1e-4)
    gate, up = act(R, M), act(R, M)
    out_rm = [torch.empty(R, M, device=dev, dtype=dt) for _ in range(3)]
    out_rd = torch.empty(R, D, device=dev, dtype=dt)
    ctr = _lib.tile_ctr(dev)
    wg_all, wu_all, wd_all = moe.w_gate_EDM.detach(), moe.w_up_EDM.detach(), moe.w_down_EMD.detach()

    def timed(fn):
        for _ in range(max(1, args.warmup)):
            fn()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
        torch.cuda.synchronize()
        for a, b in ev:
            a.record()
            fn()
            b.record()
        torch.cuda.synchronize()
        return statistics.median(a.elapsed_time(b) * 1000.0 for a, b in ev)

    def ours(rows):
        ne = len(rows)
        wg, wu, wd = wg_all[:ne], wu_all[:ne], wd_all[:ne]
        dwg, dwu, dwd = torch.empty_like(wg), torch.empty_like(wu), torch.empty_like(wd)
        offs = torch.tensor([0] + list(torch.tensor(rows).cumsum(0).tolist()), dtype=torch.int32, device=dev)
        ws_bytes = _lib.query("abacus_moe_down_fwd_ws_bytes", R, M, D, ne, code)
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
        return {
            "abacus_moe_gateup_fwd": lambda: call("abacus_moe_gateup_fwd", ptr(xp), ptr(wg), ptr(wu), ptr(offs), R,
                                                  D, M, ne, code, ptr(out_rm[0]), ptr(out_rm[1]), ptr(out_rm[2]), s),
            "abacus_moe_down_fwd": lambda: call("abacus_moe_down_fwd", ptr(h), ptr(wd), ptr(offs), R, M, D, ne, code,
                                                ptr(out_rd), ptr(ws), ws_bytes, s),
            "abacus_moe_down_bwd": lambda: call("abacus_moe_down_bwd", ptr(dy), ptr(wd), ptr(gate), ptr(up), ptr(h),
                                                ptr(offs), R, M, D, ne, code, ptr(out_rm[0]), ptr(out_rm[1]),
                                                ptr(dwd), ptr(ctr), s),
            "abacus_moe_gateup_bwd": lambda: call("abacus_moe_gateup_bwd", ptr(dgate), ptr(dup), ptr(wg), ptr(wu),
                                                  ptr(xp), ptr(offs), R, D, M, ne, code, ptr(out_rd), ptr(dwg),
                                                  ptr(dwu), ptr(ctr), s),
        }

    # hipBLASLt on the dense products: gate and up as one (R, D) x (D, 2M) product, the
    # backward's two data-gradient halves as one (R, 2M) x (2M, D), its weight gradients as
    # one (D, R) x (R, 2M)
    wgu = torch.cat([wg_all[0], wu_all[0]], dim=1)            # (D, 2M)
    wgu_t = wgu.t().contiguous()                               # (2M, D)
    wd_t = wd_all[0].t().contiguous()                          # (D, M)
    dgu = torch.cat([dgate, dup], dim=1)                       # (R, 2M)
    xp_t, h_t = xp.t().contiguous(), h.t().contiguous()
    o_r2m = torch.empty(R, 2 * M, device=dev, dtype=dt)
    o_d2m = torch.empty(D, 2 * M, device=dev, dtype=dt)
    o_md = torch.empty(M, D, device=dev, dtype=dt)
    blas = {
        "abacus_moe_gateup_fwd": lambda: torch.mm(xp, wgu, out=o_r2m),
        "abacus_moe_down_fwd": lambda: torch.mm(h, wd_all[0], out=out_rd),
        "abacus_moe_down_bwd": lambda: (torch.mm(dy, wd_t, out=out_rm[0]), torch.mm(h_t, dy, out=o_md)),
        "abacus_moe_gateup_bwd": lambda: (torch.mm(dgu, wgu_t, out=out_rd), torch.mm(xp_t, dgu, out=o_d2m)),
    }
    layouts = {"routing": counts, "equal": [R // E + (1 if e < R % E else 0) for e in range(E)], "one_expert": [R]}
    res = {}
    for name in GEMM_FLOPS_KINDS:
        row = {}
        for lay, rows in layouts.items():
            row[f"{lay}_us"] = round(timed(ours(rows)[name]), 1)
        row["hipblaslt_dense_us"] = round(timed(blas[name]), 1)
        fl = GEMM_FLOPS[name] * R * D * M
        for k in list(row):
            row[k.replace("_us", "_tflops")] = round(fl / row[k] / 1e6, 1)
        res[name] = row
    return {"gemm_shapes": "grouped-GEMM entry points on R rows split three ways; hipBLASLt on the dense product",
            "workload": wl.name, "R": R, "D": D, "M": M, "rows_per_expert": counts, "steps": args.steps,
            "kinds": res}


GEMM_FLOPS_KINDS = ("abacus_moe_gateup_fwd", "abacus_moe_down_fwd", "abacus_moe_down_bwd", "abacus_moe_gateup_bwd")


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: abacus_amd has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from abacus_amd import _lib
    from abacus_amd import workloads as W

    if args.workload in ("decoder_bf16", "decoder_fp32"):
        dt = torch.bfloat16 if args.workload == "decoder_bf16" else torch.float32
        print(json.dumps(bench_decoder(args, dt)), flush=True)
        return

    wl = W.ALL[args.workload]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    moe, x_cpu, target_cpu = W.build(wl)  # the workload recipe, on the host
    state = {k: v.detach().clone() for k, v in moe.state_dict().items()} if not args.no_cpu_baseline else None
    moe = moe.to(dev)
    x, target = x_cpu.to(dev), target_cpu.to(dev)
    # Training workloads run in train mode (the router's bias step included) with the bias reset
    # before every step, so every step routes as the first; forward-only workloads are inference
    # and run in eval mode, where the bias does not move (router.py:53).
    if args.vendor_gemm:
        print(json.dumps(bench_vendor_gemm(args, wl, moe, x)), flush=True)
        return
    if args.gemm_shapes:
        print(json.dumps(bench_gemm_shapes(args, wl, moe, x)), flush=True)
        return
    moe.train(wl.backward)
    bias0 = moe.router.expert_bias_E.detach().clone()

    def step():
        if wl.backward:
            moe.router.expert_bias_E.copy_(bias0)
        moe.zero_grad(set_to_none=True)
        xi = x.requires_grad_(wl.backward)
        with torch.set_grad_enabled(wl.backward):
            out = moe(xi)
        if wl.backward:
            loss = torch.nn.functional.mse_loss(out, target)  # mean((y - target)^2)
            loss.backward()
        xi.grad = None

    # Warmup; its last step (or one more step when there is no warmup) runs under a timer on every
    # entry point, which names the dominant kernel.
    for _ in range(max(0, args.warmup - 1)):
        step()
    probe = _lib.KernelTimer()
    with probe:
        step()
    dominant = max(probe.totals_ms().items(), key=lambda kv: kv[1][0])[0]
    torch.cuda.synchronize()

    # The timed region: HIP events only around the dominant kernel (every event record is a packet
    # between two kernels and delays the next by a few microseconds).
    timer = _lib.KernelTimer(only={dominant})
    t0 = time.perf_counter()
    with timer:
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = 1000.0 * elapsed / args.steps
    tokens_per_s = wl.tokens / (ms_per_step / 1000.0)
    d_ms, d_n = timer.totals_ms()[dominant]

    # After the timed region: the same steps again with events around every entry point, for the
    # per-kernel table (times there include the events' own delays between kernels only).
    full = _lib.KernelTimer()
    t1 = time.perf_counter()
    with full:
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
    full_elapsed = time.perf_counter() - t1

    # Forward-only workloads: the same eval-mode forward replayed from a HIP graph (one graph
    # launch per step instead of the forward's kernel launches and Python calls), timed over
    # as many steps; reported beside `value`, which stays the eager forward.
    graph = None
    if not wl.backward and not args.no_graph:
        from abacus_amd.graphs import GraphedForward
        gf = GraphedForward(moe, x)
        for _ in range(max(1, args.warmup)):
            gf(x)
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        for _ in range(args.steps):
            gf(x)
        torch.cuda.synchronize()
        g_ms = 1000.0 * (time.perf_counter() - t2) / args.steps
        graph = {"value": round(wl.tokens / (g_ms / 1000.0), 1), "unit": "tokens/s", "ms_per_step": round(g_ms, 4),
                 "how": "abacus_amd.graphs.GraphedForward: the eval-mode forward captured once, replayed per step"}
        del gf

    if args.calibrate_copy:
        src = torch.empty(1 << 29, dtype=torch.bfloat16, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    totals = full.totals_ms()
    R, D, M = wl.rows, wl.dim, wl.hidden
    peak_mfma = PEAK_BF16_TFLOPS if wl.dtype == torch.bfloat16 else PEAK_FP32_TFLOPS
    kernels = {}
    for name, (ms, n) in sorted(totals.items(), key=lambda kv: -kv[1][0]):
        avg_ms = ms / n
        rec = {"avg_us": round(avg_ms * 1000.0, 2), "calls": n, "share": round(ms / (full_elapsed * 1000.0), 4)}
        if name in GEMM_FLOPS:
            tf = GEMM_FLOPS[name] * R * D * M / (avg_ms / 1000.0) / 1e12
            rec.update({"tflops": round(tf, 1), "mfma_frac": round(tf / peak_mfma, 4)})
        b = hbm_bytes(wl, name)
        if b is not None:
            gbs = b / (avg_ms / 1000.0) / 1e9
            rec.update({"gbs": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4)})
        kernels[name] = rec

    gemm_ms = sum(totals[n][0] / totals[n][1] for n in GEMM_FLOPS if n in totals)
    gemm_tf = wl.gemm_flops() / (gemm_ms / 1000.0) / 1e12 if gemm_ms else 0.0
    counts = moe.router.last_routing.counts_E
    e_touched = int((counts > 0).sum()) if counts is not None else wl.n_experts
    stream_bytes = weight_stream_bytes(wl, e_touched)
    if not wl.backward and wl.rows <= 128 * wl.n_experts and dominant in stream_bytes:
        # decode-sized batches: the expert products stream the touched experts' weights
        b = stream_bytes[dominant]
        achieved = b / (d_ms / d_n / 1000.0) / 1e9
        roofline = {"kernel": dominant, "bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                    "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": None,
                    "algorithmic_per_launch": b, "experts_touched": e_touched}
        for n, nb in stream_bytes.items():
            if n in kernels:
                gbs = nb / (kernels[n]["avg_us"] / 1e6) / 1e9
                kernels[n].update({"gbs": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4)})
    elif dominant in GEMM_FLOPS:
        achieved = GEMM_FLOPS[dominant] * R * D * M / (d_ms / d_n / 1000.0) / 1e12
        traffic = measured_traffic(dominant) if wl.name == "mixtral_bf16" else None
        roofline = {"kernel": dominant, "bound": "mfma", "achieved": round(achieved, 1), "peak": peak_mfma,
                    "unit": "TFLOP/s", "frac": round(achieved / peak_mfma, 4), "traffic": traffic,
                    "traffic_source": TRAFFIC_FILE if traffic is not None else None,
                    "algorithmic_per_launch": GEMM_FLOPS[dominant] * R * D * M}
    else:
        b = hbm_bytes(wl, dominant) or 0
        achieved = b / (d_ms / d_n / 1000.0) / 1e9
        roofline = {"kernel": dominant, "bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                    "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": None,
                    "algorithmic_per_launch": b}

    result = {
        "metric": METRIC,
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if wl.dtype == torch.bfloat16 else "fp32",
        "data": (f"synthetic, the workload recipe: seed {wl.seed}, module init on the host, N(0,0.02^2) weights, "
                 "N(0,1) activations and target" + (", Zipf(1.2) selection bias" if wl.zipf_bias else "")),
        "config": {"workload": f"{wl.name}: MoE layer {'fwd+bwd, train mode' if wl.backward else 'fwd, eval mode'}, "
                               f"T={wl.tokens} "
                               f"(batch {wl.batch} x seq {wl.seq}), "
                               f"D={wl.dim}, E={wl.n_experts}, K={wl.top_k}, M={wl.hidden}",
                   "tokens": wl.tokens, "d_model": wl.dim, "n_experts": wl.n_experts, "top_k": wl.top_k,
                   "hidden": wl.hidden},
        "roofline": roofline,
        "grouped_gemm": {"tflops": round(gemm_tf, 1), "mfma_frac": round(gemm_tf / peak_mfma, 4),
                         "ms_per_step": round(gemm_ms, 4)},
        "kernels": kernels,
        "timing": {"value": "the timed steps carry HIP events only around the dominant kernel (roofline)",
                   "kernels": "HIP events around every entry point over as many further steps",
                   "kernels_pass_ms_per_step": round(1000.0 * full_elapsed / args.steps, 4)},
    }
    if graph is not None:
        result["graph_replay"] = graph
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(wl, state, x_cpu, target_cpu, args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
