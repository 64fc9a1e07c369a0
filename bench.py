"""Benchmark: compensated decode attention over the compressed KV cache on one MI355X.

Workload (BASELINE config c3): batch 8, 32 heads (MHA), head_dim 128, 64K
context, one query token per sequence, Q/K/V ~ N(0, 1/128) with a per-token
LogNormal(0, 0.25) factor on K and V, seed 2, cache pre-encoded (sign bits +
fp16 scale + INT4 residual + fp16 scale) and resident in HBM.  A step is one
full decode-attention pass (split kernel + combine kernel).

Prints ONE JSON line: value = achieved algorithmic HBM throughput (GB/s) over
the whole step; roofline = the split kernel alone, timed with HIP events on
the stream it runs on; cpu_baseline = the CPU oracle (PyTorch-CPU
restatement) on a bounded sample of the same heads, extrapolated to a step.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-fp16]
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

METRIC = "decode-attn µs/step + achieved HBM GB/s, 64K ctx, 32 heads, d=128, batch 8"
PEAK_HBM_GBS = 8000.0
ROOT = os.path.dirname(os.path.abspath(__file__))


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-fp16", action="store_true", help="skip the fp16 reference kernel")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="approximate CPU time budget of the baseline sample")
    ap.add_argument("--probe", action="store_true",
                    help="counter pass for rocprofv3 --pmc: one 1 GiB device copy (calibration) "
                         "then --steps attention steps, no timing output")
    return ap.parse_args()


def traffic_from_profiles():
    """HBM bytes per launch of the split kernel from the committed rocprofv3
    --pmc summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel factor),
    or None if no summary is present."""
    path = os.path.join(ROOT, "profiles", "attn_mfma_kernel_c3_counters.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read())
    return float(m.group(1)) if m else None


def cpu_baseline(q, kb, kr, vb, vr, B, H, S, d, budget_s):
    """Time the CPU oracle on whole (b, h) heads of the same workload until the
    budget is used; extrapolate to the B*H heads of one step."""
    import numpy as np
    import torch
    sys.path.insert(0, ROOT)
    from oracle import oracle as O

    n = B * H * S
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    cores = torch.get_num_threads()

    def head(b, h):
        lo = (b * H + h) * S
        def sl(blob, per, scale_off):
            return blob
        kbw = kb[lo * d // 8:(lo + S) * d // 8].cpu().view(torch.int32).view(S, d // 32)
        ks = kb[n * d // 8 + 2 * lo:n * d // 8 + 2 * (lo + S)].cpu().view(torch.float16)
        kc = kr[lo * d // 2:(lo + S) * d // 2].cpu().view(S, d // 2)
        krs = kr[n * d // 2 + 2 * lo:n * d // 2 + 2 * (lo + S)].cpu().view(torch.float16)
        vbw = vb[lo * d // 8:(lo + S) * d // 8].cpu().view(torch.int32).view(S, d // 32)
        vs = vb[n * d // 8 + 2 * lo:n * d // 8 + 2 * (lo + S)].cpu().view(torch.float16)
        vc = vr[lo * d // 2:(lo + S) * d // 2].cpu().view(S, d // 2)
        vrs = vr[n * d // 2 + 2 * lo:n * d // 2 + 2 * (lo + S)].cpu().view(torch.float16)

        def codes(c):
            c = c.to(torch.int16)
            lo_ = c & 0xF
            hi_ = (c >> 4) & 0xF
            lo_ = torch.where(lo_ >= 8, lo_ - 16, lo_)
            hi_ = torch.where(hi_ >= 8, hi_ - 16, hi_)
            return torch.stack([lo_, hi_], dim=-1).reshape(S, d).to(torch.int8)
        w64 = lambda w: w.to(torch.int64) & 0xFFFFFFFF
        return (q[b, h].cpu(), w64(kbw), ks, codes(kc), krs, w64(vbw), vs, codes(vc), vrs)

    heads = [(b, h) for b in range(B) for h in range(H)]
    rng = np.random.default_rng(0)
    order = [heads[i] for i in rng.permutation(len(heads))]
    done, t_total = 0, 0.0
    for (b, h) in order:
        args = head(b, h)               # decode of the device blobs: not timed
        t0 = time.perf_counter()
        O.compensated_attention_torch_cpu(*args)
        t_total += time.perf_counter() - t0
        done += 1
        if t_total >= budget_s or done >= len(heads):
            break
    per_head = t_total / done
    step_s = per_head * B * H
    return {
        "value": round(step_s * 1e6, 1),
        "unit": "us/step (extrapolated)",
        "gbps": round(2 * B * H * S * 84 / step_s / 1e9, 3),
        "cores": cores,
        "kind": "port",
        "sample": f"{done} of {B * H} (b,h) heads of the c3 step at full 64K context, "
                  f"PyTorch-CPU oracle, {t_total:.1f} s measured, x{B * H / done:.1f} extrapolated",
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: every box here has a single MI355X "
              f"(asked for --gpus {args.gpus}); see DESIGN.md for how the path shards.",
              file=sys.stderr)
        sys.exit(2)
    import torch
    sys.path.insert(0, ROOT)
    import bitcache_amd
    from bitcache_amd import _C
    from bitcache_amd import workloads as W
    bitcache_amd._require_extension()
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)

    cfg = W.CONFIGS["c3"]
    B, H, S, d = cfg.batch, cfg.n_heads, cfg.seq_len, cfg.head_dim
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    q, k, v = W.make_qkv(cfg, device=dev)
    kb, kr = _C.encode_fused(k.view(-1, d), False)
    vb, vr = _C.encode_fused(v.view(-1, d), False)
    if args.no_fp16:
        del k, v
    torch.cuda.synchronize()

    alg_bytes = 2 * B * H * S * W.algorithmic_bytes_per_key(d) + 2 * B * H * d * 2

    def step():
        return _C.attention(q, kb, kr, vb, vr, B, H, H, S, S, d)

    if args.probe:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        src.fill_(1)
        torch.cuda.synchronize()
        dst.copy_(src)                  # reads and writes exactly 1 GiB
        torch.cuda.synchronize()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        print(json.dumps({"probe": "done", "copy_bytes": 1 << 30, "attention_steps": args.steps}))
        return

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / args.steps

    # split kernel alone (attention_partial launches only attn_mfma_kernel), HIP
    # events on the current stream, which is the stream the kernel runs on
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.steps)]
    for i in range(args.steps):
        ev[i][0].record()
        ws = _C.attention_partial(q, kb, kr, vb, vr, B, H, H, S, S, d)
        ev[i][1].record()
        _C.attention_combine(ws, B, H, H, S, d)
    torch.cuda.synchronize()
    split_ms = sorted(a.elapsed_time(b) for a, b in ev)[len(ev) // 2]
    split_bytes = 2 * B * H * S * W.algorithmic_bytes_per_key(d)
    achieved = split_bytes / (split_ms * 1e-3) / 1e9

    fp16 = None
    if not args.no_fp16:
        for _ in range(3):
            _C.reference_attention(q, k, v, B, H, H, S, d)
        torch.cuda.synchronize()
        n16 = max(5, args.steps // 5)
        t1 = time.perf_counter()
        for _ in range(n16):
            _C.reference_attention(q, k, v, B, H, H, S, d)
        torch.cuda.synchronize()
        t16 = (time.perf_counter() - t1) / n16
        b16 = 2 * B * H * S * d * 2
        fp16 = {"us_per_step": round(t16 * 1e6, 1), "gbps": round(b16 / t16 / 1e9, 1),
                "frac_of_peak": round(b16 / t16 / 1e9 / PEAK_HBM_GBS, 4)}

    traffic = traffic_from_profiles()
    out = {
        "metric": METRIC,
        "value": round(alg_bytes / wall / 1e9, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3, 4),
        "us_per_step": round(wall * 1e6, 1),
        "tokens_per_s": round(B / wall, 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "c3: compensated decode attention, pre-encoded binary+INT4 cache",
                   "batch": B, "heads": H, "kv_heads": H, "seq_len": S, "head_dim": d,
                   "bytes_per_step": alg_bytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": traffic, "kernel": "attn_mfma_kernel<128,1,COMP>",
                     "kernel_us": round(split_ms * 1e3, 1)},
        "fp16_reference": fp16,
        "speedup_vs_fp16": (round(fp16["us_per_step"] / (wall * 1e6), 3) if fp16 else None),
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(q, kb, kr, vb, vr, B, H, S, d, args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
