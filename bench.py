"""Benchmark: the 48-block PairFormer trunk at N=768 in bf16 on one MI355X.

A step is one forward pass of the whole trunk (z [1,768,768,128],
s [1,768,384] ~ N(0,1) from seed 3, 38 of 768 tokens padded at random, 48 blocks with
their own random weights) through the HIP kernels, inputs and weights resident in HBM.
Prints one JSON line (the last line of stdout); progress goes to stderr.

Besides the metric it reports:
  roofline      the dominant kernel's achieved rate against the MI355X dense bf16 MFMA peak
                (2.5 PFLOP/s), from HIP events recorded around each of its launches on the
                launch stream (pf_kernel_timer_*: end timestamp to end timestamp) over a second
                pass of the same trunk steps; the headline pass runs with the timer off;
  block_ms      one PairFormer block (pair and single halves, one stream), median of 20;
  trunk_fp32_stream_ms  the same trunk with an fp32 residual stream and bf16 GEMM operands
                under bf16 autocast (the reference's inference regime, scripts/inference.py:803-806);
  kernels       per-kernel figures at the configuration each is quoted on: the triangle
                contraction K2 at BASELINE config 3 (N=1024) against the 50 % MFMA target, the
                other trimul kernels there, LayerNorm+transpose at N=768 against 8 TB/s, the
                flash attention at config 5 (N=2048), and one block at the reference's
                production width (c_pair=256, 8 pair heads; configs/stage0.yaml:54-56);
  gpu_eager     the same trunk as plain PyTorch eager ops (the oracle restatement of the
                reference block) on the same GPU, bf16 weights and stream under bf16
                autocast, timed like the reference harness (scripts/bench_kernels.py:107-127:
                warmup, then the median of the timed runs);
  cpu_baseline  the oracle in fp32 on the host cores: one block at N=768 (rows chunked),
                one warmup and the median of three, extrapolated x48, reported as a baseline only.
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

MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def block_flops(n: int, c: int = 128, cs: int = 384, h: int = 4, d: int = 32, hs: int = 16) -> dict[str, float]:
    """Algorithmic FLOPs of one PairFormer block at N tokens, by kernel family."""
    m = n * n
    trimul = 2 * m * c * 4 * c + 2 * 2 * m * c * c + 2 * n**3 * c  # K1 + K3 + K2
    attn_proj = 2 * m * c * (4 * h * d + h)
    attn_core = 4 * n**3 * h * d  # QK^T and PV
    attn_out = 2 * m * h * d * c
    pair_tr = 2 * m * c * 8 * c + 2 * m * 4 * c * c
    s2p = 2 * m * c * hs
    single_attn = 2 * n * cs * 4 * cs + 4 * n * n * cs + 2 * n * cs * cs
    single_tr = 2 * n * cs * 8 * cs + 2 * n * 4 * cs * cs
    return {
        "trimul": 2.0 * trimul,
        "tri_attn_core": 2.0 * attn_core,
        "attn_proj_out": 2.0 * (attn_proj + attn_out),
        "pair_transition": float(pair_tr),
        "single": float(s2p + single_attn + single_tr),
    }


# Per-launch algorithmic FLOPs of each timed kernel site, at N tokens.
def kernel_launch_flops(kernel: str, n: int) -> float:
    m, c = n * n, 128
    return {
        "tri_attn": 4.0 * n**3 * 4 * 32,
        "trimul_contract": 2.0 * n**3 * c,
        "trimul_project": 2.0 * m * c * 4 * c,
        "trimul_output": 2.0 * 2 * m * c * c,
        # A1 projects q, k, v and the 4-head pair bias; the gate GEMM runs in A3 beside
        # the output projection.
        "attn_project": 2.0 * m * c * (3 * 128 + 4),
        "attn_out": 2.0 * 2 * m * c * c,
        "pair_transition": 2.0 * m * c * 8 * c + 2.0 * m * 4 * c * c + 2.0 * m * c * 16,
    }[kernel]


def time_site(_lib, site: str, run, iters: int, warm: int = 1) -> tuple[float, int]:
    """Average duration (ms) of the launches of kernel site ``site`` over ``iters`` calls of
    ``run`` (after ``warm`` untimed calls), from HIP events on each launch's own stream."""
    import torch

    for _ in range(warm):
        run()
    torch.cuda.synchronize()
    _lib.kernel_timer_start(site)
    for _ in range(iters):
        run()
    torch.cuda.synchronize()
    total, count = _lib.kernel_timer_read()
    _lib.kernel_timer_stop()
    return total / max(count, 1), count


def kernel_figures(_lib, W, ops, attention, kernels, dev) -> list[dict]:
    """Standalone per-kernel timings at the configurations the targets are quoted on."""
    import torch

    out = []

    def entry(kernel, config, avg_ms, count, work, unit, peak, work_unit):
        rate = work / (avg_ms * 1e-3) / (1e12 if unit == "TFLOP/s" else 1e9) if count else 0.0
        out.append({
            "kernel": kernel, "config": config, "avg_launch_ms": round(avg_ms, 4), "launches": count,
            work_unit: work, "achieved": round(rate, 1), "unit": unit, "peak": peak, "frac": round(rate / peak, 4),
        })  # fmt: skip
        log(f"kernel {kernel} [{config}]: {avg_ms * 1e3:.1f} us, {rate:.1f} {unit} ({rate / peak:.3f} of peak)")

    # triangle multiplication out then in, N=1024, bf16, full mask.
    n = 1024
    sd = W.make_block_weights(2)
    mods = []
    for prefix, cls in (("tri_mul_out.", ops.TriangleMulOutgoing), ("tri_mul_in.", ops.TriangleMulIncoming)):
        m = cls(128).to(dev)
        m.load_state_dict({k[len(prefix):]: v for k, v in sd.items() if k.startswith(prefix)})
        mods.append(m.to(torch.bfloat16))
    z = torch.randn((1, n, n, 128), generator=torch.Generator().manual_seed(2)).to(dev, torch.bfloat16)
    mask = torch.ones((1, n, n), device=dev)

    def trimul():
        for m in mods:
            m.forward_residual_(z, mask)

    with torch.no_grad():
        # Kernels called right after an idle GPU run up to ~15 % slower over the first ~20
        # calls (measured on the kernel trace): each site is timed after ten untimed calls.
        for site in ("trimul_contract", "trimul_project", "trimul_output"):
            avg, cnt = time_site(_lib, site, trimul, 5, warm=10)
            entry(site, "config 3: N=1024 bf16, out+in", avg, cnt, kernel_launch_flops(site, n), "TFLOP/s",
                  MFMA_BF16_PEAK_TFLOPS, "flops_per_launch")  # fmt: skip
    del z, mods
    torch.cuda.empty_cache()

    # LayerNorm + transpose at N=768 (FusedLayerNormTranspose): one read and one write of z.
    n = 768
    x = torch.randn((1, n, n, 128), generator=torch.Generator().manual_seed(3)).to(dev, torch.bfloat16)
    w, b = torch.ones(128, device=dev), torch.zeros(128, device=dev)
    with torch.no_grad():
        avg, cnt = time_site(_lib, "ln_transpose", lambda: kernels.ln_transpose(x, w, b, 1e-5, True), 10, warm=10)
    entry("ln_transpose", "N=768 bf16", avg, cnt, 2.0 * n * n * 128 * 2, "GB/s", HBM_PEAK_GBS, "bytes_per_launch")
    del x

    # triangle attention (row, then column) at N=2048, bf16, 10 % of keys masked.
    n = 2048
    sd = W.make_block_weights(4)
    z = torch.randn((1, n, n, 128), generator=torch.Generator().manual_seed(4)).to(dev, torch.bfloat16)
    keep = torch.ones(n, device=dev)
    keep[torch.randperm(n, generator=torch.Generator().manual_seed(5))[: int(round(0.1 * n))].to(dev)] = 0.0
    with torch.no_grad():
        for transpose, prefix in ((False, "pair_attn_row."), (True, "pair_attn_col.")):
            # 10 % of the keys of every attended line masked (keys run along rows in column mode)
            mask = (keep[:, None].expand(n, n) if transpose else keep[None, :].expand(n, n)).contiguous()[None]
            m = attention.GridSelfAttention(128, 4, transpose=transpose).to(dev)
            m.load_state_dict({k[len(prefix):]: v for k, v in sd.items() if k.startswith(prefix)})
            m = m.to(torch.bfloat16)
            avg, cnt = time_site(_lib, "tri_attn", lambda: m(z, mask), 2, warm=2)
            entry("tri_attn", f"config 5: N=2048 bf16, {'columns' if transpose else 'rows'}", avg, cnt,
                  kernel_launch_flops("tri_attn", n), "TFLOP/s", MFMA_BF16_PEAK_TFLOPS, "flops_per_launch")  # fmt: skip
    del z
    torch.cuda.empty_cache()

    # One block at the reference's production width: c_pair=256 with 8 pair heads of 32
    # (configs/stage0.yaml:54-56), N=768, bf16, 5 % padded tokens; pair and single halves on
    # torch's stream, timed by CUDA events around each block (median).
    n, c, h = 768, 256, 8
    evoformer = import_module_pkg("evoformer")
    blk = evoformer.PairFormerBlock(c, 384, num_pair_heads=h).eval()
    blk.load_state_dict(W.make_block_weights(7, c_pair=c, num_pair_heads=h))
    blk = blk.to(dev).to(torch.bfloat16)
    inp = W.make_inputs(n, seed=7, pad_random=int(0.05 * n), c_pair=c)
    p = inp["pair"].to(dev, torch.bfloat16)
    s1 = inp["single"].to(dev, torch.bfloat16)
    pm, sm = inp["pair_mask"].to(dev), inp["seq_mask"].to(dev)
    times = []
    with torch.no_grad():
        for i in range(6):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            blk.forward_(p, s1, pm, sm)
            b.record()
            torch.cuda.synchronize()
            if i:
                times.append(a.elapsed_time(b))
    times.sort()
    entry("pairformer_block", f"c_pair={c}, {h} pair heads, N={n} bf16", times[len(times) // 2], len(times),
          sum(block_flops(n, c=c, h=h).values()), "TFLOP/s", MFMA_BF16_PEAK_TFLOPS, "flops_per_launch")  # fmt: skip
    del blk, p, s1
    torch.cuda.empty_cache()
    return out


def import_module_pkg(name: str):
    from importlib import import_module

    return import_module(f"deepfold3_dev_amd.{name}")


def training_figures(ops, fused, evoformer, R, dev, iters: int = 5) -> list[dict]:
    """Forward and backward at the trunk's shape (N=768): the fused attention op over 768
    lines of 4 heads and the triangle multiply module (outgoing) under grad, in bf16; and one
    training step (forward and backward) of a whole PairFormerBlock under bf16 autocast with
    an fp32 pair stream, the reference's training regime (random weights, synthetic inputs).
    Times from CUDA events on torch's stream, which the library launches on; medians over
    ``iters``."""
    import torch

    out = []

    def median_ms(fn) -> float:
        ts = []
        for _ in range(iters + 1):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b))
        return sorted(ts[1:])[len(ts[1:]) // 2]

    n, S, H, D = 768, 768, 4, 32
    g = torch.Generator().manual_seed(6)
    q, k, v = ((torch.randn(1, S, H, n, D, generator=g) * D**-0.5).to(dev, torch.bfloat16).requires_grad_(True)
               for _ in range(3))  # fmt: skip
    pb = torch.randn(1, 1, H, n, n, generator=g).to(dev).requires_grad_(True)
    rm = torch.zeros(1, S, 1, 1, n, device=dev)
    do = torch.randn(1, S, H, n, D, generator=g).to(dev, torch.bfloat16)
    state = {}

    def attn_fwd():
        state["o"] = fused._EvoformerAttention.apply(q, k, v, rm, pb, True)

    def attn_bwd():
        torch.autograd.grad(state["o"], [q, k, v, pb], grad_outputs=do, retain_graph=True)

    fwd_ms = median_ms(attn_fwd)
    bwd_ms = median_ms(attn_bwd)
    flops = 5 * 2.0 * n * n * D * S * H  # recomputed QK^T, dV, dP, dQ, dK
    rate = flops / (bwd_ms * 1e-3) / 1e12
    out.append({"op": "evo_attention backward", "config": "B=1 S=768 H=4 N=768 D=32 bf16", "fwd_ms": round(fwd_ms, 3),
                "bwd_ms": round(bwd_ms, 3), "flops": flops, "achieved": round(rate, 1), "unit": "TFLOP/s",
                "peak": MFMA_BF16_PEAK_TFLOPS, "frac": round(rate / MFMA_BF16_PEAK_TFLOPS, 4)})  # fmt: skip
    log(f"evo attention N={n}: fwd {fwd_ms:.3f} ms, bwd {bwd_ms:.3f} ms ({rate:.1f} TFLOP/s)")
    del q, k, v, pb, do, state["o"]
    torch.cuda.empty_cache()

    m = ops.TriangleMulOutgoing(128).to(dev).to(torch.bfloat16)
    for p in m.parameters():
        with torch.no_grad():
            p.copy_(torch.randn(p.shape, generator=g).to(p) / 128**0.5 if p.dim() == 2 else p)
    z = torch.randn(1, n, n, 128, generator=g).to(dev, torch.bfloat16).requires_grad_(True)
    mask = torch.ones(1, n, n, device=dev)
    gz = torch.randn(1, n, n, 128, generator=g).to(dev, torch.bfloat16)

    def tm_fwd():
        state["u"] = m(z, mask)

    def tm_bwd():
        torch.autograd.grad(state["u"], [z] + list(m.parameters()), grad_outputs=gz, retain_graph=True)

    fwd_ms = median_ms(tm_fwd)
    bwd_ms = median_ms(tm_bwd)
    out.append({"op": "TriangleMulOutgoing backward", "config": "B=1 N=768 C=128 bf16", "fwd_ms": round(fwd_ms, 3),
                "bwd_ms": round(bwd_ms, 3)})  # fmt: skip
    log(f"triangle multiply N={n}: fwd {fwd_ms:.3f} ms, bwd {bwd_ms:.3f} ms")
    del m, z, gz, state["u"]
    torch.cuda.empty_cache()

    blk = evoformer.PairFormerBlock(128, 384).to(dev)
    pair = torch.randn(1, n, n, 128, generator=g).to(dev).requires_grad_(True)
    single = torch.randn(1, n, 384, generator=g).to(dev).requires_grad_(True)
    pm, sm = torch.ones(1, n, n, device=dev), torch.ones(1, n, device=dev)
    gp = torch.randn(1, n, n, 128, generator=g).to(dev)
    gs = torch.randn(1, n, 384, generator=g).to(dev)

    def block_step():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            p, s = blk(pair, single, pm, sm)
        torch.autograd.backward([p, s], [gp, gs])
        blk.zero_grad(set_to_none=True)
        pair.grad = single.grad = None

    step_ms = median_ms(block_step)
    peak_gb = torch.cuda.max_memory_allocated() / 1e9
    log(f"PairFormerBlock training step N={n}: {step_ms:.3f} ms")

    # The same step as plain PyTorch eager ops: the oracle restatement of the reference block
    # (the eager baseline) with autograd, its four pair dropout sites fed fixed shared masks of
    # rate 0.25 (drawn once; the mask draw is not timed). It runs in fp32: under bf16 autocast
    # the backward of its batched products calls bf16 bmm on transposed views, which faults
    # the GPU on this ROCm stack.
    params = {k: v.detach().clone().requires_grad_(True) for k, v in blk.state_dict().items()}
    shape = (1, n, n, 128)
    masks = {site: R.shared_dropout_mask(shape, rowwise, 0.25, 11 + i).to(dev)
             for i, (site, rowwise) in enumerate((("tri_mul_out", True), ("tri_mul_in", True),
                                                  ("pair_attn_row", True), ("pair_attn_col", False)))}  # fmt: skip
    del blk
    torch.cuda.empty_cache()

    def eager_step():
        p, s = R.pairformer_block(pair, single, pm, sm, params, dropout=masks)
        torch.autograd.backward([p, s], [gp, gs])
        for v in params.values():
            v.grad = None
        pair.grad = single.grad = None

    torch.cuda.reset_peak_memory_stats()
    eager_ms = median_ms(eager_step)
    eager_gb = torch.cuda.max_memory_allocated() / 1e9
    out.append({"op": "PairFormerBlock training step",
                "config": "B=1 N=768 C=128, bf16 autocast, fp32 pair, training mode (pair dropout 0.25)",
                "step_ms": round(step_ms, 3), "peak_gb": round(peak_gb, 2),
                "eager_config": "oracle block ops in fp32 with autograd, same dropout rate",
                "eager_step_ms": round(eager_ms, 3), "eager_peak_gb": round(eager_gb, 2),
                "speedup": round(eager_ms / step_ms, 2)})  # fmt: skip
    log(f"eager PairFormerBlock training step N={n}: {eager_ms:.3f} ms ({eager_ms / step_ms:.2f}x the HIP step)")
    return out


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def profiled_traffic(kernel: str, n: int) -> float | None:
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3 counter summary.

    The summary (profiles/trunk_n768_bf16_hbm_traffic.md) holds FETCH_SIZE and WRITE_SIZE per
    dispatch from two counter runs of this script, scaled by a 1 GiB copy measured in the same
    runs; counters cannot be read live in the timed run.
    """
    path = os.path.join(ROOT, "profiles", f"trunk_n{n}_bf16_hbm_traffic.md")
    if not os.path.exists(path):
        return None
    key = f"traffic_bytes_per_launch {kernel}:"
    with open(path) as f:
        for line in f:
            if line.startswith(key):
                return float(line.split(":", 1)[1])
    return None


def build_stack(evoformer, W, n_blocks: int, seed: int, dev, dtype):
    import torch

    stack = evoformer.PairFormerStack(n_blocks).eval()
    sds = W.make_trunk_weights(seed, n_blocks)
    for blk, sd in zip(stack.blocks, sds):
        blk.load_state_dict(sd)
    return stack.to(dev).to(dtype), sds


def time_cpu_baseline(R, W, sds, n: int, seed: int, n_blocks: int, threads: int, runs: int) -> dict:
    import torch

    torch.set_num_threads(threads)
    inp = W.make_inputs(n, seed=seed, pad_random=int(0.05 * n))
    times = []
    with torch.no_grad():
        for i in range(runs + 1):  # the first run is the warmup
            t0 = time.perf_counter()
            R.pairformer_block(inp["pair"], inp["single"], inp["pair_mask"], inp["seq_mask"], sds[0], row_chunk=32)
            if i:
                times.append(time.perf_counter() - t0)
            log(f"cpu block run {i}/{runs} ({'warmup' if i == 0 else 'timed'})")
    times.sort()
    dt = times[len(times) // 2]
    return {
        "value": round(dt * 1e3 * n_blocks, 1),
        "unit": "ms",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "cpu_model": cpu_model(),
        "os_cpu_count": os.cpu_count(),
        "sample": f"1 of {n_blocks} blocks at N={n}, fp32 oracle on the host CPU (attention rows in chunks "
        f"of 32): one warmup, median of {runs} runs = {dt:.2f} s (runs {', '.join(f'{t:.2f}' for t in times)} s), "
        f"extrapolated x{n_blocks}",
    }


def time_gpu_eager(R, W, sds, inp, n_blocks: int, dev, steps: int, block_iters: int) -> dict:
    """Eager trunk: one warmup trunk, then the median of ``steps`` timed trunks; eager block:
    the median of ``block_iters`` runs of block 0 (after the warm trunk)."""
    import torch

    blocks = [{k: v.to(dev, torch.bfloat16) for k, v in sd.items()} for sd in sds]
    pair = inp["pair"].to(dev, torch.bfloat16)
    single = inp["single"].to(dev, torch.bfloat16)
    pm, sm = inp["pair_mask"].to(dev), inp["seq_mask"].to(dev)

    def trunk():
        p, s = pair, single
        for blk in blocks:
            p, s = R.pairformer_block(p, s, pm, sm, blk)
        return p

    def median_ms(fn, n):
        times = []
        for _ in range(n):
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
        times.sort()
        return times[len(times) // 2] * 1e3

    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        trunk()  # warmup
        torch.cuda.synchronize()
        trunk_ms = median_ms(trunk, steps)
        block_ms = median_ms(lambda: R.pairformer_block(pair, single, pm, sm, blocks[0]), block_iters)
    return {"ms": round(trunk_ms, 2), "blocks_timed": n_blocks, "warmup": 1, "steps": steps, "statistic": "median",
            "block_ms": round(block_ms, 3), "block_iters": block_iters}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--blocks", type=int, default=48)
    ap.add_argument("--n", type=int, default=768)
    ap.add_argument("--seed", type=int, default=3)
    ap.add_argument("--roofline-kernel", default="tri_attn")
    ap.add_argument("--no-eager", action="store_true", help="skip the GPU eager baseline")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--eager-steps", type=int, default=5, help="timed eager trunks (median)")
    ap.add_argument("--eager-block-iters", type=int, default=20, help="timed eager blocks (median)")
    ap.add_argument("--cpu-runs", type=int, default=3, help="timed CPU blocks after one warmup (median)")
    ap.add_argument(
        "--cpu-threads", type=int, default=0,
        help="host threads for the CPU baseline (0: torch's default, which follows OMP_NUM_THREADS)",
    )  # fmt: skip
    ap.add_argument("--no-kernels", action="store_true", help="skip the per-kernel figures")
    ap.add_argument("--no-fp32-stream", action="store_true", help="skip the fp32-stream trunk")
    ap.add_argument("--calibration-copy", action="store_true", help="run one 1 GiB copy (for PMC byte scaling)")
    ap.add_argument(
        "--kernels-only", action="store_true",
        help="run only the per-kernel figures (no trunk) and print them as one JSON line, for profiling",
    )  # fmt: skip
    ap.add_argument(
        "--training", action="store_true",
        help="run only the training-path figures (forward and backward at N=768) as one JSON line",
    )  # fmt: skip
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(
            "bench.py measures the PairFormer trunk on one GPU only: this build has no multi-GPU path "
            "(the reference shards nothing; see the sharding plan in the design notes). Run with --gpus 1.",
            file=sys.stderr,
        )
        return 2

    import torch

    import __graft_entry__

    __graft_entry__.load_package()
    from importlib import import_module

    from oracle import pairformer_ref as R

    W = import_module("deepfold3_dev_amd.weights")
    evoformer = import_module("deepfold3_dev_amd.evoformer")
    ops = import_module("deepfold3_dev_amd.ops")
    attention = import_module("deepfold3_dev_amd.attention")
    kernels = import_module("deepfold3_dev_amd.kernels")
    _lib = import_module("deepfold3_dev_amd._lib")
    if not torch.cuda.is_available():
        log("no GPU visible")
        return 1
    dev = torch.device("cuda:0")
    n, nb = args.n, args.blocks

    def calibration_copy():
        # A plain 1 GiB device-to-device copy: under `rocprofv3 --pmc FETCH_SIZE` (or
        # WRITE_SIZE) its counter value per byte scales the kernels' readings to bytes.
        buf = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        buf.clone()
        torch.cuda.synchronize()
        del buf

    if args.training:
        fused = import_module("deepfold3_dev_amd.fused")
        print(json.dumps({"training": training_figures(ops, fused, evoformer, R, dev)}), flush=True)
        return 0

    if args.kernels_only:
        if args.calibration_copy:
            calibration_copy()
        kern = kernel_figures(_lib, W, ops, attention, kernels, dev)
        print(json.dumps({"kernels": kern}), flush=True)
        return 0

    log(f"building {nb} blocks (seed {args.seed}) and inputs N={n}")
    stack, sds = build_stack(evoformer, W, nb, args.seed, dev, torch.bfloat16)
    inp = W.make_inputs(n, seed=args.seed, pad_random=int(0.05 * n))
    pair = inp["pair"].to(dev, torch.bfloat16)
    single = inp["single"].to(dev, torch.bfloat16)
    pm, sm = inp["pair_mask"].to(dev), inp["seq_mask"].to(dev)

    if args.calibration_copy:
        calibration_copy()

    out = None
    with torch.no_grad():
        for i in range(args.warmup):
            out = stack(pair, single, pm, sm)
            torch.cuda.synchronize()
            log(f"warmup {i + 1}/{args.warmup} done")
        del out
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            out = stack(pair, single, pm, sm)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        ms = (t1 - t0) * 1e3 / args.steps
        finite = bool(torch.isfinite(out[0]).all().item() and torch.isfinite(out[1]).all().item())
        log(f"timed {args.steps} steps: {ms:.2f} ms per trunk; outputs finite: {finite}")
        del out
        # Roofline pass: the same trunk steps again with the dominant kernel's launches timed.
        roof_steps = max(1, min(args.steps, 5))
        _lib.kernel_timer_start(args.roofline_kernel)
        t0 = time.perf_counter()
        for _ in range(roof_steps):
            out = stack(pair, single, pm, sm)
        torch.cuda.synchronize()
        roof_ms = (time.perf_counter() - t0) * 1e3 / roof_steps
        k_ms, k_count = _lib.kernel_timer_read()
        _lib.kernel_timer_stop()
        del out
    log(f"roofline pass ({roof_steps} trunks, {args.roofline_kernel} timed): {roof_ms:.2f} ms per trunk, "
        f"{args.roofline_kernel} {k_ms / max(k_count, 1) * 1e3:.1f} us per launch over {k_count} launches")

    # One block, pair and single halves on one stream (the median of 20 in-place runs).
    with torch.no_grad():
        p1, s1 = pair.clone(), single.clone()
        blk = stack.blocks[0]

        def one_block():
            blk.forward_(p1, s1, pm, sm)

        one_block()
        torch.cuda.synchronize()
        bt = []
        for _ in range(20):
            t_0 = time.perf_counter()
            one_block()
            torch.cuda.synchronize()
            bt.append(time.perf_counter() - t_0)
        bt.sort()
        block_ms = bt[len(bt) // 2] * 1e3
        del p1, s1
    log(f"one block: {block_ms:.3f} ms (median of 20)")

    fp32_stream = None
    if not args.no_fp32_stream:
        # The reference's inference regime: fp32 parameters and residual stream, bf16 GEMM
        # operands under autocast (scripts/inference.py:803-806).
        stack32, _ = build_stack(evoformer, W, nb, args.seed, dev, torch.float32)
        p32, s32 = inp["pair"].to(dev), inp["single"].to(dev)
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            stack32(p32, s32, pm, sm)
            torch.cuda.synchronize()
            t_0 = time.perf_counter()
            for _ in range(3):
                o32 = stack32(p32, s32, pm, sm)
            torch.cuda.synchronize()
            fp32_stream = (time.perf_counter() - t_0) * 1e3 / 3
        del stack32, p32, s32, o32
        torch.cuda.empty_cache()
        log(f"fp32-stream trunk (bf16 GEMM operands): {fp32_stream:.2f} ms")

    kern = None
    if not args.no_kernels:
        kern = kernel_figures(_lib, W, ops, attention, kernels, dev)

    fl = block_flops(n)
    trunk_flops = nb * sum(fl.values())
    tflops = trunk_flops / (ms * 1e-3) / 1e12
    k_avg_ms = k_ms / max(k_count, 1)
    k_flops = kernel_launch_flops(args.roofline_kernel, n)
    k_tflops = k_flops / (k_avg_ms * 1e-3) / 1e12 if k_count else 0.0

    eager = None
    if not args.no_eager:
        log("timing the GPU eager baseline (oracle ops, bf16)")
        eager = time_gpu_eager(R, W, sds, inp, nb, dev, args.eager_steps, args.eager_block_iters)
        eager["speedup"] = round(eager["ms"] / ms, 2)
        log(f"gpu eager: {eager['ms']} ms per trunk, HIP speed-up x{eager['speedup']}")
        torch.cuda.empty_cache()
    cpu = None
    if not args.no_cpu:
        log("timing the CPU baseline (oracle, fp32, one block)")
        threads = args.cpu_threads if args.cpu_threads > 0 else torch.get_num_threads()
        cpu = time_cpu_baseline(R, W, sds, n, args.seed, nb, threads, args.cpu_runs)
        log(f"cpu: {cpu['sample']}")

    line = {
        "metric": "PairFormer 48-block trunk ms @N=768 bf16",
        "value": round(ms, 3),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: z, s ~ N(0,1) seed 3, random-init LeCun weights per block, 5% random token padding",
        "config": {
            "workload": f"BASELINE config 4: {nb}-block PairFormer trunk forward, N_token={n}, c_pair=128, "
            "c_single=384, bf16 stream and GEMM operands (fp32 accumulate)",
            "n_tokens": n,
            "blocks": nb,
            "batch": 1,
        },
        "block_ms": round(block_ms, 3),
        "trunk_fp32_stream_ms": None if fp32_stream is None else round(fp32_stream, 2),
        "tflops": round(tflops, 1),
        "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
        "roofline": {
            "kernel": args.roofline_kernel,
            "bound": "mfma",
            "achieved": round(k_tflops, 1),
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(k_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "avg_launch_ms": round(k_avg_ms, 4),
            "launches": k_count,
            "timing": f"HIP events around each launch on its stream, end to end, second pass of {roof_steps} trunks "
            f"({round(roof_ms, 2)} ms each)",
            "flops_per_launch": k_flops,
            "traffic": profiled_traffic(args.roofline_kernel, n),
            "traffic_source": "profiles/trunk_n768_bf16_hbm_traffic.md (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-scaled)",
        },
        "kernels": kern,
        "cpu_baseline": cpu,
        "gpu_eager": eager,
        "outputs_finite": finite,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
