#!/usr/bin/env python3
"""Benchmark of the MTP speculative verify path on one MI355X.

Workload ("C3"): 27B-shaped Qwen3.5-style hybrid
model (64 layers, 3 DeltaNet : 1 GQA, hidden 5120, GQA 24Q/4KV x 256, DeltaNet
48v/16qk x 128, SwiGLU 17408, vocab 248320, 1 MTP layer), random-init bf16
weights ~ N(0, 0.02) generated on the device, batch 1, 1024-token uniform
random prompt, greedy speculative decode with MTP depth 1 (k=1, verify T=2).

A "step" is one speculative round: MTP draft -> verify forward of k+1 rows
-> fused argmax/accept -> (on a mismatch) correction forward + MTP recovery.
The headline decode covers the configured 256 new tokens (context 1024 ->
1280): --warmup untimed rounds, then --steps rounds spread evenly over the
rest of the decode are timed, one round per engine call (every round ends
with its host read, so the host clock brackets exactly one round).
`value` = committed tokens per second over the timed rounds, inputs and
weights resident in HBM, at the acceptance the reference quotes its
speculative run at (95 % at width 1): random weights accept almost no MTP
proposal, so the proposals of that leg are the model's own greedy
continuation with 5 % of positions perturbed (every round still runs the MTP
draft forward; the emitted tokens are checked equal to greedy decoding).
The rounds with the MTP head's own proposals are reported under
natural_acceptance.  Also reported: verify steps/s (one verify forward +
accept, HIP events), the HBM roofline of the dominant kernel (the skinny
GEMM), the C1 decode (tiny model, GPU and CPU oracle), and the CPU oracle
timed on the host cores and on one core (extrapolated from one layer of each
kind; see cpu_baseline.sample).
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
# HBM traffic / algorithmic weight bytes of the verify-step GEMMs (rocprofv3 FETCH_SIZE x 2.0 +
# WRITE_SIZE, scaled by a known-size copy): profiles/gemm_bf16_kernel_c3_traffic.txt
GEMM_TRAFFIC_RATIO = 1.0038
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
                 ctx: int, budget_s: float = 10.0) -> dict:
    """Times the CPU oracle on one DeltaNet layer, one GQA layer, lm_head and
    the MTP fc at the 27B shape for T=2 and T=1, and extrapolates to one
    speculative round with the GPU run's mix: with OpenMP on this host's
    cores (the reported value) and on one core (one_core)."""
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as orc  # cpu_baseline leg only

    all_cores = orc.set_threads(0)
    res = _cpu_round_estimate(orc, tokens_per_round, draft_per_round, corrections_per_round, ctx, budget_s)
    res["cores"] = all_cores
    orc.set_threads(1)
    try:
        one = _cpu_round_estimate(orc, tokens_per_round, draft_per_round, corrections_per_round, ctx, budget_s)
    finally:
        orc.set_threads(all_cores)
    one["cores"] = 1
    res["one_core"] = {k: one[k] for k in ("value", "unit", "cores", "verify_steps_per_s", "sample")}
    return res


def _cpu_round_estimate(orc, tokens_per_round: float, draft_per_round: float, corrections_per_round: float,
                        ctx: int, budget_s: float) -> dict:

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

    # Every item is run once to warm up, then whole passes over all items are
    # repeated until `budget_s` of CPU work is spent; each item's mean counts.
    xs = {T: (rng.standard_normal((T, H)) * 0.3).astype(np.float32) for T in (2, 1)}
    x2 = (rng.standard_normal((1, 2 * H)) * 0.3).astype(np.float32)
    items = {}
    for T in (2, 1):
        items[("dn", T)] = (deltanet_layer, (xs[T], T))
        items[("gqa", T)] = (gqa_layer, (xs[T], T))
        items[("lm", T)] = (orc.gemm, (xs[T], W(V // lm_split, H)))
    items[("fc", 1)] = (orc.gemm, (x2, W(H, 2 * H)))
    for fn, a in items.values():
        fn(*a)
    sums = {key: 0.0 for key in items}
    passes = 0
    t_start = time.perf_counter()
    while passes < 200 and (passes < 2 or time.perf_counter() - t_start < budget_s):
        for key, (fn, a) in items.items():
            t0 = time.perf_counter()
            fn(*a)
            sums[key] += time.perf_counter() - t0
        passes += 1
    measured = time.perf_counter() - t_start
    t = {key: v / passes for key, v in sums.items()}
    for T in (2, 1):
        t[("lm", T)] *= lm_split
    t_fc = t[("fc", 1)]
    verify = 48 * t[("dn", 2)] + 16 * t[("gqa", 2)] + t[("lm", 2)]
    fwd1 = 48 * t[("dn", 1)] + 16 * t[("gqa", 1)] + t[("lm", 1)]
    draft = t_fc + t[("gqa", 1)] + t[("lm", 1)]
    round_s = draft_per_round * draft + verify + corrections_per_round * fwd1
    return {
        "value": tokens_per_round / round_s,
        "unit": "tok/s",
        "kind": "port",
        "sample": ("CPU oracle at the 27B shape, one DeltaNet layer + one GQA layer (ctx %d) + lm_head + MTP fc, "
                   "T=2 and T=1, mean of %d passes (%.1f s of CPU work; lm_head on V/16 rows x16); extrapolated "
                   "x48/x16 to one speculative round (draft + verify T=2 + correction T=1) with the GPU run's mix"
                   % (ctx, passes, measured)),
        "verify_steps_per_s": 1.0 / verify,
        "extrapolated": True,
    }


def c1_decode(hai, E, cpu: bool) -> dict:
    """BASELINE.json configs[0] ("C1"): the tiny hybrid model (4 layers,
    hidden 256, vocab 4096), bf16 N(0, 0.02) weights of seed 0, a 32-token
    uniform random prompt, 64 new tokens, speculative decode with MTP depth
    1 -- the whole decode on the GPU engine and, in the cpu leg, on the CPU
    oracle (all cores and one core), whose tokens must be identical."""
    P, NEW = 32, 64
    prompt = E.synthetic_prompt(0, P, E.TINY["vocab"])
    eng = E.Engine(E.TINY, max_context=P + 3 * NEW + 32, max_verify_tokens=16)
    try:
        eng.init_synthetic(seed=0, std=0.02)
        eng.speculative(prompt, NEW, 1)  # warm-up
        t0 = time.perf_counter()
        toks, st, _ = eng.speculative(prompt, NEW, 1)
        gpu_s = time.perf_counter() - t0
    finally:
        eng.close()
    res = {"workload": "C1: tiny hybrid (4 layers 3 DeltaNet:1 GQA, H256, vocab 4096), 32-token prompt, 64 new "
                       "tokens, MTP k=1, bf16 N(0,0.02) weights seed 0",
           "tokens": int(len(toks)), "gpu_tok_s": round(len(toks) / gpu_s, 2), "gpu_seconds": round(gpu_s, 4),
           "acceptance_rate": round(st["accepted"] / max(1, st["proposed"]), 4)}
    if cpu:
        sys.path.insert(0, str(ROOT))
        from oracle import oracle as orc  # cpu_baseline leg only
        ref = orc.Model(orc.TINY, seed=0)
        try:
            all_cores = orc.set_threads(0)
            for cores in (all_cores, 1):
                orc.set_threads(cores)
                t0 = time.perf_counter()
                rt, _, _ = ref.speculative(prompt, NEW, 1)
                dt = time.perf_counter() - t0
                key = "cpu_oracle" if cores == all_cores else "cpu_oracle_one_core"
                res[key] = {"tok_s": round(len(rt) / dt, 2), "seconds": round(dt, 4), "cores": cores}
                res["tokens_identical"] = bool(np.array_equal(np.asarray(rt), np.asarray(toks)))
            orc.set_threads(all_cores)
        finally:
            ref.close()
    return res


def c2_ops(hai, reps: int = 50, cpu: bool = True) -> dict:
    """Op-level verify micro-bench ("C2"): batch 1,
    q_len 4, bf16 in / fp32 accumulate, tensors ~ N(0, 1), seed 1.
    GQA: 24 Q / 4 KV heads, head_dim 256, KV cache 4096 whose last 4 rows are
    the new tokens.  DeltaNet: 48 v / 16 qk heads of 128, fp32 state
    48x128x128; A_log = dt_bias = 0 so decay = sigmoid(-a) and beta =
    sigmoid(b) are sigmoids of N(0, 1).  Each kernel is launched `reps` times
    back to back between two HIP events; GB/s uses the algorithmic bytes
    (KV read; state read + write).  The CPU oracle runs the same op once."""
    import ctypes
    sys.path.insert(0, str(ROOT))
    k = hai.kernels()
    rng = np.random.default_rng(1)

    def bf(shape):
        return hai.bf16_bits(rng.standard_normal(shape).astype(np.float32)).reshape(shape)

    def dev(a):
        return hai.DeviceBuffer.from_array(np.ascontiguousarray(a))

    def timed(launch):
        e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
        hai.check(k.hai_event_create(ctypes.byref(e0)), "event")
        hai.check(k.hai_event_create(ctypes.byref(e1)), "event")
        launch()
        hai.check(k.hai_event_record(e0, None), "event")
        for _ in range(reps):
            launch()
        hai.check(k.hai_event_record(e1, None), "event")
        hai.check(k.hai_event_synchronize(e1), "event")
        ms = ctypes.c_float()
        hai.check(k.hai_event_elapsed_ms(e0, e1, ctypes.byref(ms)), "event")
        k.hai_event_destroy(e0)
        k.hai_event_destroy(e1)
        return ms.value * 1e3 / reps

    out = {}
    # ---- GQA verify over a 4096-entry cache
    T, nq, nkv, D, L = 4, 24, 4, 256, 4096
    q, g, kc, vc = bf((T, nq, D)), bf((T, nq, D)), bf((L, nkv, D)), bf((L, nkv, D))
    dq, dg, dkc, dvc = dev(q), dev(g), dev(kc), dev(vc)
    dout = hai.DeviceBuffer(T * nq * D * 2)
    dsc = hai.DeviceBuffer(k.hai_gqa_scratch_bytes(1, T, nq, D, L))
    us = timed(lambda: hai.check(k.hai_gqa_verify_bf16(dout.ptr, dq.ptr, dg.ptr, dkc.ptr, dvc.ptr, L, dsc.ptr, 1, T,
                                                        nq, nkv, D, None, L, L, None), "gqa"))
    gqa_bytes = 2 * L * nkv * D * 2
    out["gqa_verify"] = {"us": round(us, 2), "bytes": gqa_bytes, "gb_s": round(gqa_bytes / us / 1e3, 1)}
    # the same op in tolerance mode (matrix cores, P in bf16), as the batched configurations run it
    dsc_m = hai.DeviceBuffer(k.hai_gqa_mfma_scratch_bytes(1, T, nq, D, L))
    us = timed(lambda: hai.check(k.hai_gqa_verify_mfma_bf16(dout.ptr, dq.ptr, dg.ptr, dkc.ptr, dvc.ptr, L, dsc_m.ptr,
                                                             1, T, nq, nkv, D, None, L, L, None), "gqa mfma"))
    out["gqa_verify_mfma"] = {"us": round(us, 2), "bytes": gqa_bytes, "gb_s": round(gqa_bytes / us / 1e3, 1)}
    # ---- DeltaNet recurrence (reference contract: state [48][128][128] in place)
    nk, nv, dk, dv = 16, 48, 128, 128
    kw, vw = nk * dk, nv * dv
    dqk = [dev(bf((T, kw))) for _ in range(2)]
    dv_, dz = dev(bf((T, vw))), dev(bf((T, vw)))
    da, db = dev(bf((T, nv))), dev(bf((T, nv)))
    zeros = dev(np.zeros(nv, np.uint16))
    dnw = dev(bf((dv,)))
    state = (rng.standard_normal((nv, dk, dv)) * 0.1).astype(np.float32)
    dstate, dout2 = dev(state), hai.DeviceBuffer(T * vw * 2)
    us = timed(lambda: hai.check(k.hai_deltanet_recurrent_bf16(dout2.ptr, dstate.ptr, dqk[0].ptr, dqk[1].ptr, dv_.ptr,
                                                                da.ptr, db.ptr, zeros.ptr, zeros.ptr, dnw.ptr, dz.ptr,
                                                                T, nk, nv, dk, dv, 1e-6, None), "deltanet"))
    st_bytes = 2 * nv * dk * dv * 4
    out["deltanet_recurrent"] = {"us": round(us, 2), "bytes": st_bytes, "gb_s": round(st_bytes / us / 1e3, 1)}
    # ---- fused verify kernel of the engine (conv + recurrence + gated norm, state after every token kept)
    C = 2 * kw + vw
    Nin = C + vw + 2 * nv
    dproj, dcw = dev(bf((T, Nin))), dev(bf((C, 4)))
    ring, nslots = 32, T + 1
    dring = dev(np.zeros((ring, C), np.uint16))
    dslots = dev(np.zeros((nslots, nv, dk * dv), np.float32))
    us = timed(lambda: hai.check(k.hai_deltanet_verify_bf16(dout2.ptr, vw, dproj.ptr, Nin, 0, C, C + vw, C + vw + nv,
                                                             dcw.ptr, dring.ptr, ring, dslots.ptr, nslots, 1, zeros.ptr,
                                                             zeros.ptr, dnw.ptr, None, 3, 1, T, nk, nv, dk, dv, 4, 1e-6,
                                                             None), "deltanet verify"))
    fused_bytes = (1 + T) * nv * dk * dv * 4
    out["deltanet_verify_fused"] = {"us": round(us, 2), "bytes": fused_bytes, "gb_s": round(fused_bytes / us / 1e3, 1)}
    # the same with each head's value columns over several blocks (the engine's path at one sequence)
    wsb = k.hai_deltanet_workspace_bytes(1, nv, dv)
    dws = hai.DeviceBuffer(wsb)
    dws.zero()
    us = timed(lambda: hai.check(k.hai_deltanet_verify_ws_bf16(dout2.ptr, vw, dproj.ptr, Nin, 0, C, C + vw, C + vw + nv,
                                                                dcw.ptr, dring.ptr, ring, dslots.ptr, nslots, 1,
                                                                zeros.ptr, zeros.ptr, dnw.ptr, None, 3, 1, T, nk, nv, dk,
                                                                dv, 4, 1e-6, dws.ptr, wsb, None), "deltanet split"))
    out["deltanet_verify_split"] = {"us": round(us, 2), "bytes": fused_bytes, "gb_s": round(fused_bytes / us / 1e3, 1)}
    if cpu:
        from oracle import oracle as orc  # cpu_baseline leg only
        f = lambda a: hai.bf16_to_f32(a).reshape(a.shape)
        t0 = time.perf_counter()
        orc.attention(f(q), f(g), f(kc), f(vc), T, L, nq, nkv, D)
        out["gqa_verify"]["cpu_us"] = round((time.perf_counter() - t0) * 1e6, 1)
        t0 = time.perf_counter()
        orc.deltanet_recurrent(f(bf((T, kw))), f(bf((T, kw))), f(bf((T, vw))), f(bf((T, nv))), f(bf((T, nv))),
                               f(bf((T, vw))), np.zeros(nv, np.float32), np.zeros(nv, np.float32), f(bf((dv,))),
                               state, T, nk, nv, dk, dv)
        out["deltanet_recurrent"]["cpu_us"] = round((time.perf_counter() - t0) * 1e6, 1)
        out["cpu_threads"] = os.cpu_count()
    return out


def run_decode(hai, E, args, fp8: bool, steps: int):
    """Engine on the 27B shape (bf16 or FP8 weights): prefill, warmup rounds,
    `steps` timed speculative rounds, then the verify-step profile."""
    cfg = E.QWEN27B
    P, NEW = args.prompt, args.new
    tag = "fp8" if fp8 else "bf16"
    t0 = time.perf_counter()
    eng = E.Engine(cfg, max_context=P + NEW + 32, max_verify_tokens=16, use_graphs=args.graphs, fp8=fp8,
                   prefill_rows=args.prefill_rows)
    eng.init_synthetic(seed=0, std=0.02)
    hai.synchronize()
    log(f"[{tag}] engine up: {eng.weight_bytes() / 1e9:.2f} GB weights in HBM, {time.perf_counter() - t0:.1f}s")
    prompt = E.synthetic_prompt(0, P, cfg["vocab"])
    prefill = {"tokens": P}
    if not fp8:
        # the prompt through the verify step (16 rows at a time, bit-exact), then the fast prefill
        eng.set_prefill_rows(0)
        t0 = time.perf_counter()
        eng.prefill(prompt, NEW)
        prefill["verify_path_s"] = round(time.perf_counter() - t0, 4)
        prefill["verify_path_tok_s"] = round(P / prefill["verify_path_s"], 1)
        eng.set_prefill_rows(args.prefill_rows)
    t0 = time.perf_counter()
    eng.prefill(prompt, NEW)
    prefill_s = time.perf_counter() - t0
    prefill.update({"rows_per_chunk": args.prefill_rows, "seconds": round(prefill_s, 4),
                    "tok_s": round(P / prefill_s, 1)})
    log(f"[{tag}] prefill of {P} tokens: {prefill_s:.3f}s in chunks of {args.prefill_rows} rows"
        + (f" (verify path {prefill['verify_path_s']:.2f}s)" if "verify_path_s" in prefill else ""))

    out = np.zeros(NEW, np.int32)
    n0, _ = eng.spec_rounds(args.warmup, args.width, out)
    hai.synchronize()
    t0 = time.perf_counter()
    n1, st = eng.spec_rounds(steps, args.width, out)
    hai.synchronize()
    dt = time.perf_counter() - t0
    rounds = st["rounds"]
    emitted = n1 - n0
    if rounds <= 0 or emitted <= 0:
        raise RuntimeError("no speculative rounds ran (increase --new)")
    value = emitted / dt
    log(f"[{tag}] timed {rounds} rounds, {emitted} tokens in {dt:.3f}s -> {value:.2f} tok/s "
        f"(accepted {st['accepted']}/{st['proposed']})")
    prof = eng.profile_verify(args.width + 1, args.profile_iters)
    verify_ms = prof["verify_ms"]
    gemm_gbs = prof["gemm_bytes"] / (prof["gemm_ms"] * 1e-3) / 1e9
    step_gbs = prof["step_bytes"] / (verify_ms * 1e-3) / 1e9
    log(f"[{tag}] verify step {verify_ms:.3f} ms ({step_gbs:.0f} GB/s of {prof['step_bytes'] / 1e9:.2f} GB), "
        f"GEMM {prof['gemm_ms']:.3f} ms over {prof['gemm_launches']:.0f} launches ({gemm_gbs:.0f} GB/s), "
        f"draft {prof['draft_ms']:.3f} ms")
    forced = None
    if not fp8 and not args.natural_only:
        forced = run_forced(hai, eng, E, args, prompt, tag)
    eng.close()
    return value, dt, rounds, emitted, st, prof, prefill, forced


def sample_rounds(eng, width: int, out: np.ndarray, warm: int, steps: int) -> dict:
    """Runs a prefilled engine's decode to its end, one speculative round per
    call (every call ends with the round's host read, so the host clock
    brackets exactly one round): `warm` untimed rounds, then every remaining
    round, of which `steps`, evenly spaced over the rest of the decode, are
    the timed sample.  Returns the sample and the whole post-warmup decode."""
    n_prev, _ = eng.spec_rounds(warm, width, out)
    times, toks, acc, prop = [], [], [], []
    while True:
        t0 = time.perf_counter()
        n, st = eng.spec_rounds(1, width, out)
        dt = time.perf_counter() - t0
        if st["rounds"] == 0:
            break
        times.append(dt)
        toks.append(n - n_prev)
        acc.append(st["accepted"])
        prop.append(st["proposed"])
        n_prev = n
    R = len(times)
    if R == 0:
        raise RuntimeError("no speculative rounds after the warmup (increase --new or lower --warmup)")
    k = min(steps, R)
    idx = sorted({min(R - 1, int((i + 0.5) * R / k)) for i in range(k)})
    t_s, n_s = sum(times[i] for i in idx), sum(toks[i] for i in idx)
    return {"rounds": len(idx), "tokens": n_s, "seconds": t_s, "value": n_s / t_s,
            "accepted": sum(acc[i] for i in idx), "proposed": sum(prop[i] for i in idx),
            "all_rounds": R, "all_tokens": sum(toks), "all_seconds": sum(times),
            "all_accepted": sum(acc), "all_proposed": sum(prop), "emitted": n_prev}


def perturbed(g: np.ndarray, frac: float, vocab: int, seed: int = 7) -> np.ndarray:
    """A token sequence with a fraction `frac` of its positions (never the
    first) replaced by another id."""
    rng = np.random.default_rng(seed)
    d = g.copy()
    flip = rng.random(d.shape) < frac
    flip[..., 0] = False
    d[flip] = (d[flip] + 1 + rng.integers(0, vocab - 1, int(flip.sum()))) % vocab
    return d


def run_forced(hai, eng, E, args, prompt, tag: str) -> dict:
    """The headline leg, at the acceptance the reference quotes its
    speculative run at (95 % at width 1, benchmark/performance.txt:244-254):
    random weights accept almost no MTP proposal, so the proposals are the
    model's own greedy continuation with a fraction --forced-perturb of its
    positions changed (a mismatch there is rejected and corrected).  Every
    round still runs the MTP draft forward, the verify forward, the accept
    and (after a rejection) the correction; only the proposed token comes
    from the device copy of the override.  The decode covers the configured
    --new tokens (context P -> P + new): --warmup untimed rounds, then
    --steps rounds spread evenly over the rest are timed."""
    cfg = E.QWEN27B
    new = args.new
    g = eng.greedy(prompt, new)
    if len(g) < new:
        raise RuntimeError("greedy continuation ended early")
    eng.prefill(prompt, new)
    eng.set_draft_override(perturbed(g, args.forced_perturb, cfg["vocab"]))
    out = np.zeros(new, np.int32)
    r = sample_rounds(eng, args.width, out, args.warmup, args.steps)
    eng.set_draft_override(None)
    if not np.array_equal(out[:r["emitted"]], g[:r["emitted"]]):
        raise RuntimeError("forced-acceptance decode differs from greedy decoding")
    acc = r["accepted"] / max(1, r["proposed"])
    log(f"[{tag}] forced acceptance, {new}-token decode: {r['rounds']} of {r['all_rounds']} rounds after "
        f"{args.warmup} warmup timed, {r['tokens']} tokens in {r['seconds']:.3f}s -> {r['value']:.2f} tok/s "
        f"(accepted {r['accepted']}/{r['proposed']} = {acc:.3f}; whole decode "
        f"{r['all_tokens'] / r['all_seconds']:.2f} tok/s), tokens == greedy")
    return {"value": round(r["value"], 3), "unit": "tok/s", "rounds": r["rounds"], "tokens": r["tokens"],
            "seconds": round(r["seconds"], 4), "ms_per_round": round(r["seconds"] / r["rounds"] * 1e3, 4),
            "acceptance_rate": round(acc, 4), "tokens_per_round": round(r["tokens"] / r["rounds"], 4),
            "perturbed_fraction": args.forced_perturb, "tokens_equal_greedy": True,
            "decode": {"new_tokens": new, "context": [len(prompt), len(prompt) + new], "warmup_rounds": args.warmup,
                       "rounds_after_warmup": r["all_rounds"], "tokens": r["all_tokens"],
                       "tok_s": round(r["all_tokens"] / r["all_seconds"], 3),
                       "acceptance_rate": round(r["all_accepted"] / max(1, r["all_proposed"]), 4)}}


def run_batch(hai, E, args, name: str, B: int, P: int, NEW: int, width: int, fp8: bool, rounds: int) -> dict:
    """A batched configuration of BASELINE.json (C4 / C5): B sequences of
    P-token synthetic prompts decoded in lockstep speculative rounds; GEMMs
    of 4 or more rows run on the MFMA GEMMs (tolerance mode).  Two legs over
    the whole NEW-token decode, each with `rounds` timed rounds spread over
    it after two warmup rounds: the MTP head's own proposals (random weights
    accept none), then forced acceptance -- the proposals are each
    sequence's continuation from the first leg (speculative greedy decoding
    is lossless, so that is the sequence's greedy continuation) with
    --forced-perturb of the positions changed, so that partial acceptance
    and the per-sequence state rollback are timed."""
    cfg = E.QWEN27B
    t0 = time.perf_counter()
    cap = P + (width + 2) * NEW + 32
    prows = min(args.batch_prefill_rows, P)
    eng = E.Engine(cfg, max_context=cap, max_verify_tokens=16, fp8=fp8, batch=B, mfma=True, prefill_rows=prows)
    eng.init_synthetic(seed=0, std=0.02)
    hai.synchronize()
    log(f"[{name}] engine up: B={B}, {eng.weight_bytes() / 1e9:.2f} GB weights, {time.perf_counter() - t0:.1f}s")
    prompts = np.stack([E.synthetic_prompt(b, P, cfg["vocab"]) for b in range(B)])
    t0 = time.perf_counter()
    eng.prefill(prompts, NEW)
    hai.synchronize()
    prefill_s = time.perf_counter() - t0
    log(f"[{name}] prefill of {B} x {P} tokens: {prefill_s:.2f}s ({B * P / prefill_s:.0f} tok/s)")
    out = np.zeros((B, NEW), np.int32)
    nat = sample_rounds(eng, width, out, 2, rounds)
    prof = eng.profile_verify(width + 1, 3)
    natural = out.copy()
    gemm_gbs = prof["gemm_bytes"] / (prof["gemm_ms"] * 1e-3) / 1e9
    step_gbs = prof["step_bytes"] / (prof["verify_ms"] * 1e-3) / 1e9
    res = {
        "workload": f"{name}: 27B shape, batch {B} x {P}-token prompts, MTP k={width}, {NEW} new tokens per "
                    f"sequence, {'FP8 E4M3 128x128-block weights' if fp8 else 'bf16 weights'}; GEMMs of 4 or more "
                    f"rows (verify, correction, draft) on the MFMA GEMMs (FP8 codes decoded to bf16 in LDS)",
        "value": round(nat["value"], 2), "unit": "tok/s (all sequences)", "rounds": nat["rounds"],
        "ms_per_round": round(nat["seconds"] / nat["rounds"] * 1e3, 3),
        "verify_ms": round(prof["verify_ms"], 3), "verify_rows": B * (width + 1),
        "verify_bytes": round(prof["step_bytes"]), "verify_hbm_frac": round(step_gbs / HBM_PEAK_GBS, 4),
        "gemm_gb_s": round(gemm_gbs, 1), "gemm_launches": prof["gemm_launches"],
        "draft_ms": round(prof["draft_ms"], 3), "prefill_s": round(prefill_s, 3),
        "prefill_tok_s": round(B * P / prefill_s, 1), "prefill_rows_per_chunk": prows,
        "acceptance_rate": round(nat["accepted"] / max(1, nat["proposed"]), 4),
    }
    log(f"[{name}] natural proposals: {nat['tokens']} tokens in {nat['seconds']:.2f}s over {nat['rounds']} sampled "
        f"rounds -> {res['value']} tok/s; verify {prof['verify_ms']:.2f} ms ({step_gbs:.0f} GB/s), "
        f"GEMM {gemm_gbs:.0f} GB/s, draft {prof['draft_ms']:.2f} ms")
    if not args.natural_only:
        eng.prefill(prompts, NEW)
        eng.set_draft_override(perturbed(natural, args.forced_perturb, cfg["vocab"]))
        out = np.zeros((B, NEW), np.int32)
        fr = sample_rounds(eng, width, out, 2, rounds)
        eng.set_draft_override(None)
        same = [bool(np.array_equal(out[b], natural[b])) for b in range(B)]
        acc = fr["accepted"] / max(1, fr["proposed"])
        res["forced"] = {
            "value": round(fr["value"], 2), "unit": "tok/s (all sequences)", "rounds": fr["rounds"],
            "tokens": fr["tokens"], "ms_per_round": round(fr["seconds"] / fr["rounds"] * 1e3, 3),
            "acceptance_rate": round(acc, 4), "tokens_per_round": round(fr["tokens"] / fr["rounds"], 3),
            "perturbed_fraction": args.forced_perturb,
            "decode_tok_s": round(fr["all_tokens"] / fr["all_seconds"], 2),
            "decode_acceptance_rate": round(fr["all_accepted"] / max(1, fr["all_proposed"]), 4),
            "sequences_equal_natural": sum(same),
        }
        log(f"[{name}] forced acceptance: {fr['tokens']} tokens in {fr['seconds']:.2f}s over {fr['rounds']} sampled "
            f"rounds -> {fr['value']:.2f} tok/s (accepted {fr['accepted']}/{fr['proposed']} = {acc:.3f}; "
            f"whole decode {res['forced']['decode_tok_s']} tok/s); {sum(same)}/{B} sequences equal the first leg's")
    eng.close()
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20,
                    help="timed speculative rounds of the headline leg, spread evenly over its decode")
    ap.add_argument("--warmup", type=int, default=5, help="untimed rounds before the timed ones")
    ap.add_argument("--natural-rounds", type=int, default=20,
                    help="timed rounds with the MTP head's own proposals (natural_acceptance)")
    ap.add_argument("--prompt", type=int, default=1024)
    ap.add_argument("--prefill-rows", type=int, default=1024,
                    help="prompt rows per fast-prefill chunk of the bs=1 engines (the verify-path prefill is "
                         "timed beside it)")
    ap.add_argument("--batch-prefill-rows", type=int, default=1024,
                    help="prompt rows per sequence and fast-prefill chunk of the C4 / C5 engines (C4 8 x 8192: "
                         "512 rows 3.85 s, 1024 rows 3.60 s, 2048 rows 3.57 s)")
    ap.add_argument("--new", type=int, default=256)
    ap.add_argument("--width", type=int, default=1)
    ap.add_argument("--profile-iters", type=int, default=5)
    ap.add_argument("--natural-only", action="store_true",
                    help="skip the forced-acceptance legs (the line's value then comes from the natural rounds)")
    ap.add_argument("--forced-perturb", type=float, default=0.05,
                    help="fraction of the greedy continuation's positions changed in the forced drafts")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--graphs", action="store_true",
                    help="replay captured HIP graphs (rocprofv3 kernel tracing cannot follow graph launches)")
    ap.add_argument("--no-fp8", action="store_true",
                    help="skip the FP8-weight leg (C5 weight format at batch 1, reported under fp8_weights)")
    ap.add_argument("--fp8-steps", type=int, default=60)
    ap.add_argument("--no-c4", action="store_true",
                    help="skip C4 (batch 8 x 8192-token prompts, k=3; reported under batch_c4)")
    ap.add_argument("--no-c5", action="store_true",
                    help="skip C5 (FP8 weights, batch 32 x 512-token prompts, k=1; reported under batch_c5)")
    ap.add_argument("--batch-rounds", type=int, default=12,
                    help="timed rounds of each C4 / C5 leg, spread evenly over the decode")
    ap.add_argument("--no-c1", action="store_true", help="skip the C1 tiny-model decode (reported under c1)")
    ap.add_argument("--no-c2", action="store_true", help="skip the C2 op micro-bench (reported under c2_ops)")
    ap.add_argument("--c4-prompt", type=int, default=8192,
                    help="C4 prompt length (8192 is the configuration; shorter only for counter passes)")
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

    P, NEW = args.prompt, args.new
    nat_value, dt, rounds, emitted, st, prof, prefill, forced = run_decode(hai, E, args, fp8=False,
                                                                            steps=args.natural_rounds)
    verify_ms = prof["verify_ms"]
    gemm_gbs = prof["gemm_bytes"] / (prof["gemm_ms"] * 1e-3) / 1e9
    step_gbs = prof["step_bytes"] / (verify_ms * 1e-3) / 1e9

    # The line's value: the forced-acceptance leg (the acceptance the
    # reference quotes, 95 % at width 1) when it ran, else the natural rounds.
    if forced is not None:
        value, v_rounds, v_tokens, v_ms = forced["value"], forced["rounds"], forced["tokens"], forced["ms_per_round"]
        drafts = ("MTP draft forward every round, proposals replaced by the model's own greedy continuation with "
                  "%.0f%% of positions perturbed (acceptance %.3f; tokens checked equal to greedy decoding); "
                  "the whole %d-token decode runs, %d rounds after %d warmup rounds timed, spread evenly over it"
                  % (100 * args.forced_perturb, forced["acceptance_rate"], NEW, forced["rounds"], args.warmup))
    else:
        value, v_rounds, v_tokens, v_ms = nat_value, rounds, emitted, dt / rounds * 1e3
        drafts = "the MTP head's own proposals (random weights: acceptance %.3f)" % (st["accepted"] / max(1, st["proposed"]))
    result = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": v_rounds,
        "warmup": args.warmup,
        "ms_per_step": round(v_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init bf16 weights ~N(0,0.02) generated on device, uniform random prompt ids)",
        "config": {
            "workload": "C3: 27B-shape hybrid (64 layers 3 DeltaNet:1 GQA, H5120, vocab 248320, 1 MTP layer), "
                        "bs=1, %d-token prompt, greedy speculative decode MTP k=%d" % (P, args.width),
            "prompt_tokens": P, "new_tokens": NEW, "timed_tokens": v_tokens, "mtp_k": args.width, "batch": 1,
            "drafts": drafts,
        },
        "natural_acceptance": {
            "value": round(nat_value, 3), "unit": "tok/s", "rounds": rounds, "tokens": emitted,
            "ms_per_round": round(dt / rounds * 1e3, 4),
            "acceptance_rate": round(st["accepted"] / max(1, st["proposed"]), 4),
        },
        "verify_steps_per_s": round(1e3 / verify_ms, 3),
        "verify_ms": round(verify_ms, 4),
        "verify_hbm_frac": round(step_gbs / HBM_PEAK_GBS, 4),
        "draft_ms": round(prof["draft_ms"], 4),
        "acceptance_rate": forced["acceptance_rate"] if forced else round(st["accepted"] / max(1, st["proposed"]), 4),
        "decode": forced["decode"] if forced else None,
        "tokens_per_round": round(v_tokens / v_rounds, 4),
        "prefill": prefill,
        "roofline": {
            "bound": "hbm",
            "achieved": round(gemm_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gemm_gbs / HBM_PEAK_GBS, 4),
            # HBM bytes per launch: the live algorithmic bytes x the FETCH_SIZE + WRITE_SIZE
            # ratio measured by rocprofv3 on the same kernels at the C3 shapes
            # (profiles/gemm_bf16_kernel_c3_traffic.txt; counters cannot be read inside this run)
            "traffic": round(prof["gemm_bytes"] / prof["gemm_launches"] * GEMM_TRAFFIC_RATIO),
            "traffic_ratio": GEMM_TRAFFIC_RATIO,
            "kernel": "gemm_bf16_kernel (skinny bf16 GEMM, verify T=%d)" % (args.width + 1),
            "bytes_per_launch": round(prof["gemm_bytes"] / prof["gemm_launches"]),
            "ms_per_launch": round(prof["gemm_ms"] / prof["gemm_launches"], 5),
        },
    }
    if not args.no_fp8:
        fv, fdt, frounds, femitted, fst, fprof, _, _ = run_decode(hai, E, args, fp8=True, steps=args.fp8_steps)
        fgemm = fprof["gemm_bytes"] / (fprof["gemm_ms"] * 1e-3) / 1e9
        fstep = fprof["step_bytes"] / (fprof["verify_ms"] * 1e-3) / 1e9
        result["fp8_weights"] = {
            "workload": "C3 shape with the C5 weight format: QuantizedWeight Linears FP8 E4M3, 128x128 fp32 "
                        "block scales U(0.5,2)/448, quantised from the bf16 init; embed, lm_head, MTP fc, "
                        "in_proj_a/b bf16; bs=1, MTP k=%d" % args.width,
            "value": round(fv, 3), "unit": "tok/s", "steps": frounds,
            "ms_per_step": round(fdt / frounds * 1e3, 4),
            "verify_ms": round(fprof["verify_ms"], 4),
            "verify_steps_per_s": round(1e3 / fprof["verify_ms"], 3),
            "verify_bytes": round(fprof["step_bytes"]),
            "verify_hbm_frac": round(fstep / HBM_PEAK_GBS, 4),
            "gemm_gb_s": round(fgemm, 1), "gemm_hbm_frac": round(fgemm / HBM_PEAK_GBS, 4),
            "gemm_launches": fprof["gemm_launches"],
            "draft_ms": round(fprof["draft_ms"], 4),
            "acceptance_rate": round(fst["accepted"] / max(1, fst["proposed"]), 4),
        }
    # The batched configurations are extra fields; an error there (raised by
    # the engine, not a device fault) is recorded without losing the line.
    for flag, key, run in ((args.no_c4, "batch_c4", ("C4", 8, args.c4_prompt, 128, 3, False)),
                           (args.no_c5, "batch_c5", ("C5", 32, 512, 128, 1, True))):
        if flag:
            continue
        try:
            result[key] = run_batch(hai, E, args, *run[:5], run[5], args.batch_rounds)
        except RuntimeError as e:
            result[key] = {"error": str(e)}
            log(f"[{run[0]}] failed: {e}")
    if not args.no_c1:
        result["c1"] = c1_decode(hai, E, cpu=not args.no_cpu_baseline)
        log("C1: " + json.dumps(result["c1"]))
    if not args.no_c2:
        result["c2_ops"] = c2_ops(hai, cpu=not args.no_cpu_baseline)
        log("C2 ops: " + ", ".join(f"{k} {v['us']} us ({v['gb_s']} GB/s)" for k, v in result["c2_ops"].items()
                                   if isinstance(v, dict)))
    if not args.no_cpu_baseline:
        t0 = time.perf_counter()
        # the CPU oracle extrapolated to the same round mix as `value`
        mix = forced if forced is not None else None
        tpr = mix["tokens_per_round"] if mix else emitted / rounds
        acc = mix["acceptance_rate"] if mix else st["accepted"] / max(1, st["proposed"])
        result["cpu_baseline"] = cpu_baseline(tpr, args.width, args.width * (1.0 - acc), P + NEW)
        log(f"cpu baseline leg: {time.perf_counter() - t0:.1f}s")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
