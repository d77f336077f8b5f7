#!/usr/bin/env python3
"""Benchmark of the MTP speculative verify path on one MI355X.

Workload ("C3"): 27B-shaped Qwen3.5-style hybrid
model (64 layers, 3 DeltaNet : 1 GQA, hidden 5120, GQA 24Q/4KV x 256, DeltaNet
48v/16qk x 128, SwiGLU 17408, vocab 248320, 1 MTP layer), random-init bf16
weights ~ N(0, 0.02) generated on the device, batch 1, 1024-token uniform
random prompt, greedy speculative decode with MTP depth 1 (k=1, verify T=2).

A "step" is one speculative round: MTP draft -> verify forward of k+1 rows
-> fused argmax/accept -> (on a mismatch) correction forward + MTP recovery.
`value` = committed (accepted) tokens per second over the timed rounds, inputs
and weights resident in HBM.  Also reported: verify steps/s (one verify
forward + accept, HIP events), the HBM roofline of the dominant kernel (the
skinny GEMM), and the CPU oracle timed on the host cores (extrapolated from
one layer of each kind; see cpu_baseline.sample).
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
HBM_PEAK_GBS = 8000.0
METRIC = "accepted tok/s + verify steps/s (27B-shape bf16, bs=1, MTP k=1); % HBM peak"


def load_package():
    name = "hybridai_amd"
    if name in sys.modules:
        return sys.modules[name]
    pkg = ROOT / "vicold.hybridai_amd"
    spec = importlib.util.spec_from_file_location(name, pkg / "__init__.py", submodule_search_locations=[str(pkg)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(tokens_per_round: float, draft_per_round: float, corrections_per_round: float,
                 ctx: int) -> dict:
    """Times the CPU oracle (OpenMP, this host's cores) on one DeltaNet layer,
    one GQA layer, lm_head and the MTP fc at the 27B shape for T=2 and T=1,
    and extrapolates to one speculative round with the GPU run's mix."""
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as orc  # cpu_baseline leg only

    cfg = orc.QWEN27B
    H, F, V = cfg["hidden"], cfg["ffn"], cfg["vocab"]
    nq, nkv, D, R = cfg["num_q_heads"], cfg["num_kv_heads"], cfg["head_dim"], cfg["rope_dim"]
    nk, nv, dk, dv = cfg["lin_qk_heads"], cfg["lin_v_heads"], cfg["lin_k_dim"], cfg["lin_v_dim"]
    C, vw, qw, kvw = 2 * nk * dk + nv * dv, nv * dv, nq * D, nkv * D
    rng = np.random.default_rng(0)
    block = (rng.standard_normal(1 << 20) * 0.02).astype(np.float32)
    lm_split = 16  # lm_head timed on V/16 rows and scaled (the GEMV cost is linear in N)
    n_big = max(F * H, (C + vw + 2 * nv) * H, (V // lm_split) * H)
    big = np.tile(block, (n_big + block.size - 1) // block.size)  # one buffer serves every weight

    def W(n, k):
        return big[:n * k].reshape(n, k)

    norm_w = (rng.standard_normal(H) * 0.02).astype(np.float32)
    kc = (rng.standard_normal((ctx, nkv, D)) * 0.5).astype(np.float32)
    vc = (rng.standard_normal((ctx, nkv, D)) * 0.5).astype(np.float32)

    def mlp(x):
        xn = orc.rmsnorm(x, norm_w)
        g = orc.gemm(xn, W(F, H))
        u = orc.gemm(xn, W(F, H))
        return orc.gemm(orc.silu_mul(g, u), W(H, F))

    def deltanet_layer(x, T):
        xn = orc.rmsnorm(x, norm_w)
        p = orc.gemm(xn, W(C + vw + 2 * nv, H))
        q, k, v, _ = orc.deltanet_conv(p[:, :C], W(C, 4), np.zeros((C, 3), np.float32), T, nk, nv, dk, dv, 4)
        out, _ = orc.deltanet_recurrent(q, k, v, p[:, C + vw:C + vw + nv], p[:, C + vw + nv:], p[:, C:C + vw],
                                        norm_w[:nv], norm_w[:nv], norm_w[:dv], np.zeros((nv, dk, dv), np.float32),
                                        T, nk, nv, dk, dv)
        h = orc.add(x, orc.gemm(out, W(H, vw)))
        return orc.add(h, mlp(h))

    def gqa_layer(x, T):
        xn = orc.rmsnorm(x, norm_w)
        p = orc.gemm(xn, W(2 * qw + 2 * kvw, H))
        q, g = orc.q_gate_rmsnorm_rope(p[:, :2 * qw], norm_w[:D], T, nq, D, R, ctx - T, 1e7)
        k = orc.k_rmsnorm_rope(p[:, 2 * qw:2 * qw + kvw], norm_w[:D], T, nkv, D, R, ctx - T, 1e7)
        kc[ctx - T:] = k
        a = orc.attention(q, g, kc, vc, T, ctx, nq, nkv, D)
        h = orc.add(x, orc.gemm(a.reshape(T, qw), W(H, qw)))
        return orc.add(h, mlp(h))

    def timed(fn, *args, reps=3):
        best = float("inf")
        for _ in range(reps):
            t0 = time.perf_counter()
            fn(*args)
            best = min(best, time.perf_counter() - t0)
        return best

    t = {}
    for T in (2, 1):
        x = (rng.standard_normal((T, H)) * 0.3).astype(np.float32)
        t[("dn", T)] = timed(deltanet_layer, x, T)
        t[("gqa", T)] = timed(gqa_layer, x, T)
        t[("lm", T)] = lm_split * timed(orc.gemm, x, W(V // lm_split, H))
    x2 = (rng.standard_normal((1, 2 * H)) * 0.3).astype(np.float32)
    t_fc = timed(orc.gemm, x2, W(H, 2 * H))
    verify = 48 * t[("dn", 2)] + 16 * t[("gqa", 2)] + t[("lm", 2)]
    fwd1 = 48 * t[("dn", 1)] + 16 * t[("gqa", 1)] + t[("lm", 1)]
    draft = t_fc + t[("gqa", 1)] + t[("lm", 1)]
    round_s = draft_per_round * draft + verify + corrections_per_round * fwd1
    cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    measured = 3 * (sum(v for k, v in t.items() if k[0] != "lm") + t_fc +
                    sum(v for k, v in t.items() if k[0] == "lm") / lm_split)
    return {
        "value": tokens_per_round / round_s,
        "unit": "tok/s",
        "cores": cores,
        "kind": "port",
        "sample": ("CPU oracle at the 27B shape, one DeltaNet layer + one GQA layer (ctx %d) + lm_head + MTP fc, "
                   "T=2 and T=1, best of 3 each (%.1f s of CPU work; lm_head on V/16 rows x16); extrapolated x48/x16 to one speculative "
                   "round (draft + verify T=2 + correction T=1) with the GPU run's mix" % (ctx, measured)),
        "verify_steps_per_s": 1.0 / verify,
        "extrapolated": True,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100, help="timed speculative rounds")
    ap.add_argument("--warmup", type=int, default=8, help="untimed rounds before timing")
    ap.add_argument("--prompt", type=int, default=1024)
    ap.add_argument("--new", type=int, default=256)
    ap.add_argument("--width", type=int, default=1)
    ap.add_argument("--profile-iters", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--graphs", action="store_true",
                    help="replay captured HIP graphs (rocprofv3 kernel tracing cannot follow graph launches)")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="first run one device-to-device copy of this many bytes (the known-size reference "
                         "dispatch that scales rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the path runs on a single MI355X); "
              "multi-GPU runs are not part of it", file=sys.stderr)
        sys.exit(2)

    hai = load_package()
    from hybridai_amd import engine as E

    if args.copy_bytes > 0:
        src, dst = hai.DeviceBuffer(args.copy_bytes), hai.DeviceBuffer(args.copy_bytes)
        src.zero()
        hai.check(hai.kernels().hai_memcpy_d2d(dst.ptr, src.ptr, args.copy_bytes, None), "calibration copy")
        hai.synchronize()
        log(f"calibration copy of {args.copy_bytes} bytes done")
        del src, dst

    cfg = E.QWEN27B
    P, NEW = args.prompt, args.new
    t0 = time.perf_counter()
    eng = E.Engine(cfg, max_context=P + NEW + 32, max_verify_tokens=16, use_graphs=args.graphs)
    eng.init_synthetic(seed=0, std=0.02)
    hai.synchronize()
    log(f"engine up: {eng.weight_bytes() / 1e9:.2f} GB weights in HBM, {time.perf_counter() - t0:.1f}s")
    prompt = E.synthetic_prompt(0, P, cfg["vocab"])
    t0 = time.perf_counter()
    eng.prefill(prompt, NEW)
    prefill_s = time.perf_counter() - t0
    log(f"prefill of {P} tokens: {prefill_s:.2f}s")

    out = np.zeros(NEW, np.int32)
    n0, _ = eng.spec_rounds(args.warmup, args.width, out)
    hai.synchronize()
    t0 = time.perf_counter()
    n1, st = eng.spec_rounds(args.steps, args.width, out)
    hai.synchronize()
    dt = time.perf_counter() - t0
    rounds = st["rounds"]
    emitted = n1 - n0
    if rounds <= 0 or emitted <= 0:
        raise RuntimeError("no speculative rounds ran (increase --new)")
    value = emitted / dt
    log(f"timed {rounds} rounds, {emitted} tokens in {dt:.3f}s -> {value:.2f} tok/s "
        f"(accepted {st['accepted']}/{st['proposed']})")

    prof = eng.profile_verify(args.width + 1, args.profile_iters)
    verify_ms = prof["verify_ms"]
    gemm_gbs = prof["gemm_bytes"] / (prof["gemm_ms"] * 1e-3) / 1e9
    step_gbs = prof["step_bytes"] / (verify_ms * 1e-3) / 1e9
    log(f"verify step {verify_ms:.3f} ms ({step_gbs:.0f} GB/s of {prof['step_bytes'] / 1e9:.2f} GB), "
        f"GEMM {prof['gemm_ms']:.3f} ms over {prof['gemm_launches']:.0f} launches ({gemm_gbs:.0f} GB/s), "
        f"draft {prof['draft_ms']:.3f} ms")

    result = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": rounds,
        "warmup": args.warmup,
        "ms_per_step": round(dt / rounds * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init bf16 weights ~N(0,0.02) generated on device, uniform random prompt ids)",
        "config": {
            "workload": "C3: 27B-shape hybrid (64 layers 3 DeltaNet:1 GQA, H5120, vocab 248320, 1 MTP layer), "
                        "bs=1, %d-token prompt, greedy speculative decode MTP k=%d" % (P, args.width),
            "prompt_tokens": P, "new_tokens": NEW, "mtp_k": args.width, "batch": 1,
        },
        "verify_steps_per_s": round(1e3 / verify_ms, 3),
        "verify_ms": round(verify_ms, 4),
        "verify_hbm_frac": round(step_gbs / HBM_PEAK_GBS, 4),
        "draft_ms": round(prof["draft_ms"], 4),
        "acceptance_rate": round(st["accepted"] / max(1, st["proposed"]), 4),
        "tokens_per_round": round(emitted / rounds, 4),
        "prefill_s": round(prefill_s, 3),
        "roofline": {
            "bound": "hbm",
            "achieved": round(gemm_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gemm_gbs / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "gemm_bf16_kernel (skinny bf16 GEMM, verify T=%d)" % (args.width + 1),
            "bytes_per_launch": round(prof["gemm_bytes"] / prof["gemm_launches"]),
            "ms_per_launch": round(prof["gemm_ms"] / prof["gemm_launches"], 5),
        },
    }
    eng.close()
    if not args.no_cpu_baseline:
        t0 = time.perf_counter()
        result["cpu_baseline"] = cpu_baseline(emitted / rounds, st["proposed"] / rounds,
                                              st["corrections"] / rounds, P + NEW)
        log(f"cpu baseline leg: {time.perf_counter() - t0:.1f}s")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
