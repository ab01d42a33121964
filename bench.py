"""Speculative-decoding benchmark on one MI355X: Qwen3-8B-shaped Q4_K_M target + Qwen3-0.6B-shaped Q8_0 draft, k=4.

A step = one generation of 256 tokens (greedy, f16 KV) after a 512-token seeded prompt; the prompt's KV is cached
after the first call, so every step is pure speculative decoding (draft k tokens, verify k+1 in one target pass,
accept / roll back), as zerollm's generateSpeculative does for a repeated prompt. Weights are random-init N(0, 0.02)
of the named shapes, generated in HBM (no network, no checkpoints). Prints one JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12  # MI355X HBM3E, bytes/s
# HBM bytes per launch of the roofline kernel (k_gemv_mfma<SWIGLU>, Q4_K ffn_gate + ffn_up at M = 5): FETCH_SIZE
# and WRITE_SIZE counter runs over `bench.py --probe-only`, each scaled by the same counter's reading for a plain copy of
# known size (profiles/gemv_gate_up_m5_traffic.md). A hardware counter cannot be read inside this timed run.
ROOFLINE_TRAFFIC_BYTES = 59_219_000
PROMPT, GEN, K = 512, 256, 4


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_baseline(t_spec, d_spec, prompt, seconds, threads):
    """The reference's worker-pool path restated for this host's CPU (oracle/pool_simd.c: AVX-512 VNNI int8 tiles, f64
    combine, `threads` OpenMP workers each owning a slice of every matrix, k + 1 verify rows in one pass over the
    weights), running the same greedy speculative loop on the same weights at the same context: both models prefill the
    512-token prompt (untimed), then whole cycles run until `seconds` have passed. Its logits equal the oracle's bit for
    bit (tests/test_pool_simd.py), so it emits the tokens the GPU emits. On a CPU without AVX-512 VNNI the scalar oracle
    runs instead, at a context of 8 prompt tokens."""
    from oracle import oracle as O
    from oracle import pool as P
    from oracle.spec import feed, plain, speculative_greedy
    from zerollm_amd import synth

    simd = P.supported()
    O.set_threads(threads)
    t0 = time.perf_counter()
    models = []
    for spec in (t_spec, d_spec):
        arrays = {t.name: synth.tensor_bytes(t, use_device=True) for t in spec.tensors}
        src = O.ArraySource(spec, arrays)
        models.append(P.SimdPoolModel(src, ctx=1024, threads=threads) if simd else
                      O.OracleModel(src, ctx=64, kv="f16", threads=threads))
        del arrays
    log(f"cpu baseline: weights on host in {time.perf_counter() - t0:.1f}s ({P.cpu_name()}, "
        f"{'AVX-512 VNNI pool restatement' if simd else 'scalar oracle'}, {threads} threads)")
    tm, dm = models
    ctx_prompt = prompt if simd else prompt[-8:]
    tp = time.perf_counter()
    for m in models:
        feed(m, ctx_prompt[:-1], False)
    log(f"cpu baseline: prefill of {len(ctx_prompt) - 1} tokens into both models {time.perf_counter() - tp:.1f}s")
    ts = time.perf_counter()
    out, cycles = speculative_greedy(tm, dm, ctx_prompt, K, 256, deadline=ts + seconds)
    el = time.perf_counter() - ts
    # plain greedy decoding of the same prompt on the same target, for half as long
    tp = time.perf_counter()
    n_plain = 0
    for _ in plain(tm, ctx_prompt, len(out)):
        n_plain += 1
        if time.perf_counter() - tp > seconds / 2:
            break
    el_plain = time.perf_counter() - tp
    for m in models:
        m.close()
    if simd:
        sample = (f"AVX-512 VNNI restatement of the worker-pool path (int8 tiles, f64 combine, batched k+1 verify), greedy "
                  f"speculative decoding k={K} after the {len(prompt)}-token prompt (prefill untimed): {len(out)} tokens in "
                  f"{cycles} cycles, {el:.1f}s, f16 KV, same weights, logits bit-identical to the oracle; CPU: "
                  f"{P.cpu_name()}")
    else:
        sample = (f"scalar oracle (no AVX-512 VNNI on {P.cpu_name()}), greedy speculative decoding k={K} of {len(out)} "
                  f"tokens in {cycles} cycles, {el:.1f}s, f16 KV, context <= 40 positions, same weights")
    return {"value": round(len(out) / el, 3), "unit": "tok/s", "cores": threads, "kind": "port", "sample": sample,
            "plain_tok_s": round(n_plain / el_plain, 3),
            "plain_sample": f"plain greedy decoding of the same prompt on the same target: {n_plain} tokens in {el_plain:.1f}s"}


def _stats(v):
    v = sorted(v)
    return {"median": round(v[len(v) // 2] if len(v) % 2 else 0.5 * (v[len(v) // 2 - 1] + v[len(v) // 2]), 2),
            "min": round(v[0], 2), "max": round(v[-1], 2)}


def paired_rounds(target, draft, prompt, rounds, gen, k=K):
    """Plain greedy decoding (generate) against greedy speculative decoding (generateSpeculative) of the same prompt on
    the same models, in interleaved rounds whose order alternates, medians with min-max, as the reference's own
    comparison does (tools/specbench.mjs:67-106). Both reuse the cached prompt, so each round times decoding alone."""
    from zerollm_amd.generate import generate
    from zerollm_amd.speculative import generate_speculative

    spec, plain, ratio, acc = [], [], [], []
    ref = None
    for r in range(rounds):
        res = {}
        for mode in (("spec", "plain") if r % 2 == 0 else ("plain", "spec")):
            st = {}
            t0 = time.perf_counter()
            if mode == "spec":
                out = list(generate_speculative(target, draft, prompt, k=k, max_tokens=gen, stats=st))
                acc.append(st["speculative"]["acceptRate"])
            else:
                out = list(generate(target, prompt, max_tokens=gen, stats=st))
            res[mode] = len(out) / (time.perf_counter() - t0)
            ref = out if ref is None else ref
            assert out == ref, "greedy speculative decoding must emit the plain greedy stream"
        spec.append(res["spec"])
        plain.append(res["plain"])
        ratio.append(res["spec"] / res["plain"])
        log(f"paired round {r}: speculative {res['spec']:.1f} tok/s, plain {res['plain']:.1f} tok/s")
    return {"rounds": rounds, "tokens": gen, "speculative_tok_s": _stats(spec), "plain_tok_s": _stats(plain),
            "speedup": _stats(ratio), "accept_rate": round(sum(acc) / len(acc), 4)}


def modeled(cycle_ms, k=K):
    """Throughput the measured cycle would give at per-draft acceptance rate a: a cycle emits (1 - a^(k+1)) / (1 - a)
    tokens on average (k + 1 at a = 1), and its cost hardly depends on a (k draft passes, counting the catch-up feed of
    one or two tokens, and one (k+1)-row verify pass). The random-weight pair accepts almost nothing, so the measured
    value is the a ~ 0 point."""
    out = {}
    for a in (0.5, 0.7, 0.9, 1.0):
        e = k + 1 if a == 1.0 else (1 - a ** (k + 1)) / (1 - a)
        out[str(a)] = round(e / (cycle_ms * 1e-3), 1)
    return out


LONG_PROMPT, LONG_K = 16384, 8
PREFILL_CHUNK = 64
CLOSE_LAYER_STD, CLOSE_TAIL = 0.0003, 0.01


def long_context(args):
    """The same Qwen3-8B / 0.6B-shaped pair with the context pre-filled to 16384 seeded ids, stochastic acceptance
    (temperature 0.7, top-k 40, top-p 0.9, seeded uniforms for the accept test and residual draws) and k = 8: each verify
    pass runs 9 rows of GQA attention over a 16K-entry f16 KV cache, and rejected positions are rolled back. A step is
    one generation of `gen` tokens after the cached prompt; the sampler is re-seeded per step, so every step yields the
    same tokens."""
    from zerollm_amd import synth
    from zerollm_amd.sampler import HipSampler
    from zerollm_amd.speculative import generate_speculative

    t_spec, d_spec = synth.qwen3_8b_pair()
    ctx = LONG_PROMPT + args.gen + 2 * (LONG_K + 1)
    t0 = time.perf_counter()
    # passes of up to 64 tokens: the prompt is prefilled in 64-token chunks (every weight read once per chunk)
    target = synth.build_on_device(t_spec, ctx=ctx, kv="f16", max_batch=PREFILL_CHUNK)
    draft = synth.build_on_device(d_spec, ctx=ctx, kv="f16", max_batch=PREFILL_CHUNK)
    log(f"models built in HBM in {time.perf_counter() - t0:.1f}s (ctx {ctx})")
    prompt = synth.seeded_ids(LONG_PROMPT, 2025, t_spec.vocab)

    def run(st):
        smp = HipSampler(temperature=0.7, top_k=40, top_p=0.9, seed=1234)
        try:
            return list(generate_speculative(target, draft, prompt, k=LONG_K, max_tokens=args.gen, sample=smp, stats=st))
        finally:
            smp.close()

    t1 = time.perf_counter()
    st0 = {}
    first = run(st0)
    pf_t = (st0["prefillMs"] - st0["speculative"]["draftPrefillMs"]) / 1e3
    pf_d = st0["speculative"]["draftPrefillMs"] / 1e3
    log(f"first call (prefill {LONG_PROMPT} tokens into both models + {len(first)} tokens) {time.perf_counter() - t1:.1f}s; "
        f"prefill target {pf_t:.2f}s, draft {pf_d:.2f}s")
    for w in range(args.warmup):
        assert run({}) == first, "seeded sampling must reproduce the same tokens"
    times, cycles, acc, drafted, dms, vms, n_tok = [], 0, 0, 0, 0.0, 0.0, 0
    for s in range(args.steps):
        st = {}
        ts = time.perf_counter()
        out = run(st)
        times.append(time.perf_counter() - ts)
        assert out == first
        sp = st["speculative"]
        cycles += sp["cycles"]; acc += sp["accepted"]; drafted += sp["drafted"]; dms += sp["draftMs"]; vms += sp["verifyMs"]
        n_tok += len(out)
        log(f"step {s}: {len(out) / times[-1]:.1f} tok/s, {sp['cycles']} cycles, accept {sp['acceptRate']:.3f}")
    total = sum(times)
    kv_t = 2 * t_spec.n_layer * t_spec.n_head_kv * t_spec.head_dim * 2 * (LONG_PROMPT + args.gen // 2)
    kv_d = 2 * d_spec.n_layer * d_spec.n_head_kv * d_spec.head_dim * 2 * (LONG_PROMPT + args.gen // 2)
    line = {
        "metric": "spec-decode tok/s, Qwen3-8B-Q4_K_M + 0.6B-Q8_0 draft, k=8, T=0.7, 16K context",
        "value": round(n_tok / total, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(total * 1e3 / args.steps, 2), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "q4_k/q6_k/q8_0 weights, int8 activations, f64 combine, f16 KV",
        "data": "synthetic: random-init N(0,0.02) weights of the named shapes, seeded uniform prompt ids",
        "config": {"workload": "speculative decode with stochastic acceptance (temperature 0.7, top-k 40, top-p 0.9, "
                               "seeded uniforms), k=8, context pre-filled to 16384 seeded ids, f16 KV, same models as the "
                               "headline workload", "k": LONG_K, "prompt": LONG_PROMPT, "generate": args.gen,
                   "accept_rate": round(acc / max(1, drafted), 4), "tokens_per_cycle": round(n_tok / max(1, cycles), 3),
                   "cycle_ms": round(total * 1e3 / max(1, cycles), 3), "draft_ms_per_cycle": round(dms / max(1, cycles), 3),
                   "verify_accept_ms_per_cycle": round(vms / max(1, cycles), 3),
                   "modeled_tok_s_at_accept": modeled(total * 1e3 / max(1, cycles), LONG_K),
                   "kv_bytes_per_target_pass": kv_t, "kv_bytes_per_draft_pass": kv_d,
                   "prefill_s": {"tokens": LONG_PROMPT - 1, "chunk": PREFILL_CHUNK, "target": round(pf_t, 3),
                                 "draft": round(pf_d, 3)}},
    }
    target.close()
    draft.close()
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--gen", type=int, default=GEN, help="tokens generated per step (profiling runs use fewer)")
    ap.add_argument("--rounds", type=int, default=5,
                    help="paired rounds of plain vs speculative decoding after the timed steps (0: none)")
    ap.add_argument("--probe-only", action="store_true",
                    help="only the roofline kernel's timed launches (for hardware-counter runs); prints the roofline")
    ap.add_argument("--workload", choices=["headline", "long"], default="headline",
                    help="long: the same pair with a 16384-token context, stochastic acceptance (T 0.7, top-k 40, "
                         "top-p 0.9) and k = 8")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the speculative step runs on a single MI355X (asked for --gpus {args.gpus}); "
              "across GPUs it shards as independent sequences per GPU (data parallel), not by splitting a pass",
              file=sys.stderr)
        sys.exit(2)

    from zerollm_amd import model as M, synth
    from zerollm_amd.speculative import generate_speculative

    if args.probe_only:
        from zerollm_amd.gemv_bench import copy_calibration
        copy_calibration(256)  # a kernel of known traffic for scaling hardware byte counters (before any other launch)
    M.init(0)
    dev = M.device_info()
    log("device:", dev)
    if args.workload == "long":
        return long_context(args)
    t_spec, d_spec = synth.qwen3_8b_pair()
    t0 = time.perf_counter()
    target = synth.build_on_device(t_spec, ctx=1024, kv="f16")
    draft = synth.build_on_device(d_spec, ctx=1024, kv="f16")
    log(f"models built in HBM in {time.perf_counter() - t0:.1f}s: target {target.weight_bytes / 1e9:.3f} GB/pass, "
        f"draft {draft.weight_bytes / 1e9:.3f} GB/pass")
    prompt = synth.seeded_ids(PROMPT, 2024, t_spec.vocab)
    if args.probe_only:
        target.forward_batch(prompt[:K + 1], logits="none")
        ms, b = target.probe_gemv("gate_up", K + 1, 4 * t_spec.n_layer)
        print(json.dumps({"kernel": "k_gemv_mfma<SWIGLU> (Q4_K, M=5)", "launch_ms": round(ms, 5), "bytes_per_launch": b,
                          "GBps": round(b / (ms * 1e-3) / 1e9, 1)}), flush=True)
        target.close()
        draft.close()
        return

    t1 = time.perf_counter()
    st = {}
    first = list(generate_speculative(target, draft, prompt, k=K, max_tokens=args.gen, stats=st))
    log(f"first call (prefill {PROMPT} tokens + graph capture + {len(first)} tokens) {time.perf_counter() - t1:.1f}s")
    for w in range(args.warmup):
        out = list(generate_speculative(target, draft, prompt, k=K, max_tokens=args.gen, stats=st))
        assert out == first, "greedy output must be deterministic"
        log(f"warmup {w}: {st['speculative']['cycles']} cycles, accept {st['speculative']['acceptRate']:.3f}")
    times, cycles, acc, drafted, dms, vms = [], 0, 0, 0, 0.0, 0.0
    for s in range(args.steps):
        st = {}
        ts = time.perf_counter()
        out = list(generate_speculative(target, draft, prompt, k=K, max_tokens=args.gen, stats=st))
        times.append(time.perf_counter() - ts)
        assert out == first
        cycles += st["speculative"]["cycles"]
        acc += st["speculative"]["accepted"]
        drafted += st["speculative"]["drafted"]
        dms += st["speculative"]["draftMs"]
        vms += st["speculative"]["verifyMs"]
        log(f"step {s}: {args.gen / times[-1]:.1f} tok/s, {st['speculative']['cycles']} cycles")
    total = sum(times)
    tok_s = args.gen * args.steps / total
    # the dominant kernel of the verify pass: ffn_gate+ffn_up GEMV with SwiGLU epilogue at M = k+1, timed with HIP
    # events on the target's stream over back-to-back launches through all 36 layers' weights (2 GB: cache-cold)
    iters = 4 * t_spec.n_layer
    probe_ms, bytes_per = target.probe_gemv("gate_up", K + 1, iters)
    achieved = bytes_per / (probe_ms * 1e-3)
    others = {w: target.probe_gemv(w, K + 1, t_spec.n_layer if w != "output" else 8) for w in ("qkv", "wo", "down", "output")}
    cycle_ms = total * 1e3 / cycles
    bytes_cycle = target.weight_bytes + K * draft.weight_bytes
    line = {
        "metric": "spec-decode tok/s, Qwen3-8B-Q4_K_M + 0.6B-Q8_0 draft, k=4; verify GEMV % HBM peak",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(total * 1e3 / args.steps, 2), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "q4_k/q6_k/q8_0 weights, int8 activations, f64 combine, f16 KV",
        "data": "synthetic: random-init N(0,0.02) weights of the named shapes, seeded uniform prompt ids",
        "config": {"workload": "speculative decode, Qwen3-8B-shaped Q4_K_M target (36L d4096 32/8 heads FFN 12288 "
                               "V151936) + Qwen3-0.6B-shaped Q8_0 draft (28L d1024 16/8 heads FFN 3072), k=4, prompt 512, "
                               "256 greedy tokens per step, f16 KV",
                   "k": K, "prompt": PROMPT, "generate": args.gen, "accept_rate": round(acc / max(1, drafted), 4),
                   "tokens_per_cycle": round(args.gen * args.steps / cycles, 3), "cycle_ms": round(cycle_ms, 3),
                   "draft_ms_per_cycle": round(dms / cycles, 3), "verify_accept_ms_per_cycle": round(vms / cycles, 3),
                   "weight_bytes_per_cycle": bytes_cycle,
                   "modeled_tok_s_at_accept": modeled(cycle_ms),
                   "cycle_weight_bw_frac": round(bytes_cycle / (cycle_ms * 1e-3) / HBM_PEAK, 4)},
        "roofline": {"bound": "hbm", "kernel": "k_gemv_mfma<SWIGLU> (Q4_K ffn_gate+ffn_up, M=k+1=5, int8 dots on the matrix cores)",
                     "achieved": round(achieved / 1e9, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK, 4), "traffic": ROOFLINE_TRAFFIC_BYTES,
                     "launch_ms": round(probe_ms, 5), "bytes_per_launch": bytes_per, "launches": iters,
                     "other_gemvs_GBps": {w: round(b / (ms * 1e-3) / 1e9, 1) for w, (ms, b) in others.items()}},
    }
    speculation = {"headline_pair": paired_rounds(target, draft, prompt, args.rounds, args.gen)} if args.rounds else {}
    target.close()
    draft.close()
    if args.rounds:
        # an agreeing pair of the same shapes, formats and bytes per pass (so the same cycle cost), to measure what
        # speculation buys when the draft is accepted
        c_spec, cd_spec = synth.qwen3_8b_close_pair(layer_std=CLOSE_LAYER_STD, tail=CLOSE_TAIL)
        ct = synth.build_on_device(c_spec, ctx=1024, kv="f16")
        cd = synth.build_on_device(cd_spec, ctx=1024, kv="f16")
        list(generate_speculative(ct, cd, prompt, k=K, max_tokens=args.gen))  # prefill, graph capture
        ap = paired_rounds(ct, cd, prompt, args.rounds, args.gen)
        ap["pair"] = (f"the headline shapes and formats with per-layer matrices N(0, {CLOSE_LAYER_STD}) and the target's "
                      f"output norm weighing the 3072 embedding columns the draft lacks by {CLOSE_TAIL} "
                      "(synth.qwen3_8b_close_pair)")
        speculation["agreeing_pair"] = ap
        ct.close()
        cd.close()
    line["speculation"] = speculation
    if not args.no_cpu:
        threads = min(16, os.cpu_count() or 1)
        line["cpu_baseline"] = cpu_baseline(t_spec, d_spec, prompt, args.cpu_seconds, threads)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
