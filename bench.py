"""Benchmark: the 48-block PairFormer trunk at N=768 in bf16 on one MI355X.

A step is one forward pass of the whole trunk (z [1,768,768,128],
s [1,768,384] ~ N(0,1) from seed 3, 38 of 768 tokens padded at random, 48 blocks with
their own random weights) through the HIP kernels, inputs and weights resident in HBM.
Prints one JSON line (the last line of stdout); progress goes to stderr.

Besides the metric it reports:
  roofline      the dominant kernel's achieved rate from HIP events recorded around each
                of its launches on its own stream inside the timed region (pf_kernel_timer_*),
                against the MI355X dense bf16 MFMA peak (2.5 PFLOP/s);
  gpu_eager     the same trunk as plain PyTorch eager ops (the oracle restatement of the
                reference block) on the same GPU, bf16 weights and stream under bf16
                autocast, timed like the reference harness (scripts/bench_kernels.py:107-127);
  cpu_baseline  the oracle in fp32 on the host cores: one block at N=768 (rows chunked),
                extrapolated x48, reported as a baseline only.
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
        "attn_project": 2.0 * m * c * (4 * 128 + 4),
        "attn_out": 2.0 * m * c * c,
        "pair_transition": 2.0 * m * c * 8 * c + 2.0 * m * 4 * c * c + 2.0 * m * c * 16,
    }[kernel]


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


def time_cpu_baseline(R, W, sds, n: int, seed: int, n_blocks: int, threads: int) -> dict:
    import torch

    torch.set_num_threads(threads)
    inp = W.make_inputs(n, seed=seed, pad_random=int(0.05 * n))
    with torch.no_grad():
        t0 = time.perf_counter()
        R.pairformer_block(inp["pair"], inp["single"], inp["pair_mask"], inp["seq_mask"], sds[0], row_chunk=32)
        dt = time.perf_counter() - t0
    return {
        "value": round(dt * 1e3 * n_blocks, 1),
        "unit": "ms",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"1 of {n_blocks} blocks at N={n}, fp32 oracle on the host CPU "
        f"(attention rows in chunks of 32), {dt:.2f} s, extrapolated x{n_blocks}",
    }


def time_gpu_eager(R, W, sds, inp, n_blocks: int, dev, steps: int) -> dict:
    import torch

    blocks = [{k: v.to(dev, torch.bfloat16) for k, v in sd.items()} for sd in sds]
    pair = inp["pair"].to(dev, torch.bfloat16)
    single = inp["single"].to(dev, torch.bfloat16)
    pm, sm = inp["pair_mask"].to(dev), inp["seq_mask"].to(dev)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        R.pairformer_block(pair, single, pm, sm, blocks[0])  # warmup
        torch.cuda.synchronize()
        times = []
        for _ in range(steps):
            t0 = time.perf_counter()
            p, s = pair, single
            for blk in blocks:
                p, s = R.pairformer_block(p, s, pm, sm, blk)
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
    times.sort()
    return {"ms": round(times[len(times) // 2] * 1e3, 2), "blocks_timed": n_blocks, "steps": steps}


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
    ap.add_argument("--eager-steps", type=int, default=1)
    ap.add_argument("--cpu-threads", type=int, default=16)
    ap.add_argument("--calibration-copy", action="store_true", help="run one 1 GiB copy (for PMC byte scaling)")
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
    _lib = import_module("deepfold3_dev_amd._lib")
    if not torch.cuda.is_available():
        log("no GPU visible")
        return 1
    dev = torch.device("cuda:0")
    n, nb = args.n, args.blocks

    log(f"building {nb} blocks (seed {args.seed}) and inputs N={n}")
    stack, sds = build_stack(evoformer, W, nb, args.seed, dev, torch.bfloat16)
    inp = W.make_inputs(n, seed=args.seed, pad_random=int(0.05 * n))
    pair = inp["pair"].to(dev, torch.bfloat16)
    single = inp["single"].to(dev, torch.bfloat16)
    pm, sm = inp["pair_mask"].to(dev), inp["seq_mask"].to(dev)

    if args.calibration_copy:
        # A plain 1 GiB device-to-device copy: under `rocprofv3 --pmc FETCH_SIZE` (or
        # WRITE_SIZE) its counter value per byte scales the kernels' readings to bytes.
        buf = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        buf.clone()
        torch.cuda.synchronize()
        del buf

    out = None
    with torch.no_grad():
        for i in range(args.warmup):
            out = stack(pair, single, pm, sm)
            torch.cuda.synchronize()
            log(f"warmup {i + 1}/{args.warmup} done")
        del out
        _lib.kernel_timer_start(args.roofline_kernel)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            out = stack(pair, single, pm, sm)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        k_ms, k_count = _lib.kernel_timer_read()
        _lib.kernel_timer_stop()
    ms = (t1 - t0) * 1e3 / args.steps
    finite = bool(torch.isfinite(out[0]).all().item() and torch.isfinite(out[1]).all().item())
    log(f"timed {args.steps} steps: {ms:.2f} ms per trunk; outputs finite: {finite}")
    del out

    fl = block_flops(n)
    trunk_flops = nb * sum(fl.values())
    tflops = trunk_flops / (ms * 1e-3) / 1e12
    k_avg_ms = k_ms / max(k_count, 1)
    k_flops = kernel_launch_flops(args.roofline_kernel, n)
    k_tflops = k_flops / (k_avg_ms * 1e-3) / 1e12 if k_count else 0.0

    eager = None
    if not args.no_eager:
        log("timing the GPU eager baseline (oracle ops, bf16)")
        eager = time_gpu_eager(R, W, sds, inp, nb, dev, args.eager_steps)
        eager["speedup"] = round(eager["ms"] / ms, 2)
        log(f"gpu eager: {eager['ms']} ms per trunk, HIP speed-up x{eager['speedup']}")
        torch.cuda.empty_cache()
    cpu = None
    if not args.no_cpu:
        log("timing the CPU baseline (oracle, fp32, one block)")
        cpu = time_cpu_baseline(R, W, sds, n, args.seed, nb, min(args.cpu_threads, os.cpu_count() or 1))
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
            "flops_per_launch": k_flops,
            "traffic": profiled_traffic(args.roofline_kernel, n),
            "traffic_source": "profiles/trunk_n768_bf16_hbm_traffic.md (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-scaled)",
        },
        "cpu_baseline": cpu,
        "gpu_eager": eager,
        "outputs_finite": finite,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
