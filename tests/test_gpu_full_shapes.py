"""GPU checks at the benchmark configurations' full shapes (test/spec-logits.test.js:13-38, 97-139 and
test/spec-generate.test.js:29-59 are the reference's versions of these checks):
- the Qwen3-8B-shaped Q4_K_M target and Qwen3-0.6B-shaped Q8_0 draft (headline configuration): a 5-row verify pass
  equals 5 single-token passes bit for bit, the first verify rows of both models match the oracle, and greedy
  speculative decoding equals plain greedy decoding;
- the same pair at a 16384-token context (long-context configuration): a 9-row verify pass equals 9 single-token
  passes, rollback leaves what a fresh continuation computes, and seeded stochastic k = 8 runs reproduce;
- the Qwen3.5-4B-shaped hybrid after a 2048-token prefix: a 5-row verify pass equals 5 single-token passes (logits and
  recurrent state), and rollback by snapshot restore + replay equals the sequential state.
The oracle cannot run 16K or 2048-token contexts of these models in seconds, so there the checks are the
size-independent properties above; the oracle comparisons run on short prefixes of the same models."""
import numpy as np
import pytest

from oracle import oracle as O
from zerollm_amd import synth
from zerollm_amd.generate import generate
from zerollm_amd.sampler import HipSampler
from zerollm_amd.speculative import generate_speculative

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _oracle(spec, ctx=64):
    arrays = {t.name: synth.tensor_bytes(t, use_device=True) for t in spec.tensors}
    O.set_threads(16)
    return O.OracleModel(O.ArraySource(spec, arrays), ctx=ctx, kv="f16", threads=16)


@pytest.fixture(scope="module")
def pair_8b():
    t_spec, d_spec = synth.qwen3_8b_pair()
    return t_spec, d_spec


@pytest.mark.timeout(600)
@pytest.mark.parametrize("which", ["target", "draft"])
def test_c3_verify_rows_equal_single_passes_and_oracle(gpu, pair_8b, which):
    spec = pair_8b[0] if which == "target" else pair_8b[1]
    pre = synth.seeded_ids(4, 31, spec.vocab)
    ver = synth.seeded_ids(5, 32, spec.vocab)
    print(f"case c3 {which}: build", flush=True)
    m = synth.build_on_device(spec, ctx=64, kv="f16")
    m.forward_batch(pre, logits="none")
    rows = m.forward_batch(ver, logits="all").copy()
    m.truncate(len(pre))
    seq = np.stack([m.forward(t).copy() for t in ver])
    m.close()
    assert (_bits(rows) == _bits(seq)).all(), "a 5-row verify pass must equal 5 single-token passes bit for bit"
    print(f"case c3 {which}: oracle", flush=True)
    ref = _oracle(spec)
    for t in pre:
        ref.forward(t, logits=False)
    n_cmp = 3 if which == "target" else 5
    want = np.stack([ref.forward(t) for t in ver[:n_cmp]])
    ref.close()
    got = rows[:n_cmp]
    d = np.abs(got.astype(np.float64) - want)
    exact = np.mean(_bits(got) == _bits(want))
    print(f"c3 {which}: max-abs {d.max():.3g}, mean-abs {d.mean():.3g}, bit-exact {exact:.5f}", flush=True)
    assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS
    assert (got.argmax(1) == want.argmax(1)).all()
    assert exact >= 0.999 and d.max() <= 1e-6 * np.abs(want).max()


@pytest.mark.timeout(600)
@pytest.mark.parametrize("which", ["target", "draft"])
def test_prefill_chunks_of_64_equal_chunks_of_16(gpu, pair_8b, which):
    """Prefill in chunks of 64 tokens (each weight read once per chunk on the GEMM, score dots on the matrix cores) and
    of 16, 16 tokens through the GEMV kernels alone (ZEROLLM_GEMM_MAXM=0: two passes of 8), and token by token all
    leave the same KV cache: the next rows' logits are the same bits (prefillTokens, src/model/generate.js:18-31)."""
    import os

    spec = pair_8b[0] if which == "target" else pair_8b[1]
    ids = synth.seeded_ids(200, 41, spec.vocab)
    nxt = synth.seeded_ids(3, 42, spec.vocab)
    rows = {}
    for mb, maxm in ((1, "64"), (64, "64"), (16, "64"), (16, "0")):
        print(f"case prefill chunks {which} max_batch {mb} gemm {maxm}", flush=True)
        os.environ["ZEROLLM_GEMM_MAXM"] = maxm
        try:
            m = synth.build_on_device(spec, ctx=256, kv="f16", max_batch=mb)
            for i in range(0, len(ids), mb):
                m.forward_batch(ids[i:i + mb], logits="none")
            rows[(mb, maxm)] = np.stack([m.forward(t).copy() for t in nxt])
            m.close()
        finally:
            del os.environ["ZEROLLM_GEMM_MAXM"]
    ref = rows[(1, "64")]  # token by token: the GEMV kernels and the lane-chain scores alone
    for k, v in rows.items():
        assert (_bits(v) == _bits(ref)).all(), k


@pytest.mark.timeout(600)
def test_c3_greedy_speculative_equals_plain_greedy(gpu, pair_8b):
    t_spec, d_spec = pair_8b
    p = synth.seeded_ids(32, 2024, t_spec.vocab)
    print("case c3 speculative", flush=True)
    t = synth.build_on_device(t_spec, ctx=128, kv="f16")
    d = synth.build_on_device(d_spec, ctx=128, kv="f16")
    st = {}
    spec = list(generate_speculative(t, d, p, k=4, max_tokens=12, stats=st))
    t.reset()
    plain = list(generate(t, p, max_tokens=12))
    assert spec == plain and len(spec) == 12
    assert st["speculative"]["cycles"] >= 3
    t.close()
    d.close()


@pytest.mark.timeout(1200)
def test_sampled_cycles_at_the_full_vocabulary_match_oracle(gpu):
    """Stochastic acceptance with the long-context configuration's sampler (temperature 0.7, top-k 40, top-p 0.9, k = 8)
    on the 8B / 0.6B shapes, 151,936 logits per row: the two-stage candidate selection over 75 blocks, the acceptance
    over fixed candidate lists and the residual and bonus draws, cycle by cycle against the oracle's
    generateSpeculative (src/model/speculative.js:155-209): the same drafts, accept counts and tokens, and the same final
    mulberry32 state. The agreeing pair of the same shapes (synth.qwen3_8b_close_pair) is used so that cycles both
    accept and reject."""
    from oracle import spec as OS
    from zerollm_amd import model as Mdl

    t_spec, d_spec = synth.qwen3_8b_close_pair()
    prompt = synth.seeded_ids(6, 57, t_spec.vocab)
    cfg = dict(temperature=0.7, top_k=40, top_p=0.9)
    print("case full-vocabulary sampled cycles: device", flush=True)
    t = synth.build_on_device(t_spec, ctx=64, kv="f16")
    d = synth.build_on_device(d_spec, ctx=64, kv="f16")
    s = HipSampler(seed=1234, **cfg)
    log, st = [], {}
    out = list(generate_speculative(t, d, prompt, k=8, max_tokens=10, sample=s, stats=st, cycle_log=log))
    rng, limit = s.rng_state, Mdl.verify_limit(t)
    for x in (t, d, s):
        x.close()
    print(f"device: {len(log)} cycles {log}", flush=True)
    print("case full-vocabulary sampled cycles: oracle", flush=True)
    ot, od = _oracle(t_spec), _oracle(d_spec)
    os_ = O.Sampler(seed=1234, **cfg)
    o_log = []
    o_out = list(OS.speculative(ot, od, prompt, k=8, max_tokens=10, sample=os_, cycle_log=o_log, t_limit=limit))
    ot.close()
    od.close()
    for c, (g, w) in enumerate(zip(log, o_log)):
        assert g == w, f"cycle {c}: device {g} vs oracle {w}"
    assert log == o_log and out == o_out and rng == os_.rng.state


def test_sampler_at_the_full_vocabulary_matches_oracle(gpu, pair_8b):
    """Sampled distributions over the 151,936 logits of the 0.6B-shaped draft against the oracle sampler on the same
    logits: top_k 40 selects over the 75 blocks' candidate lists in LDS; top_k 200 and 256 have more candidates than
    LDS holds and select over the whole row."""
    d_spec = pair_8b[1]
    print("case sampler at the full vocabulary", flush=True)
    d = synth.build_on_device(d_spec, ctx=64, kv="f16")
    for cfg in [dict(temperature=0.7, top_k=40, top_p=0.9), dict(temperature=1.0, top_k=200, top_p=1.0),
                dict(temperature=1.2, top_k=256, top_p=0.95, min_p=0.01)]:
        ds = HipSampler(seed=21, **cfg)
        hs = O.Sampler(seed=21, **cfg)
        for tk in synth.seeded_ids(3, 77, d_spec.vocab):
            logits = d.forward(tk).copy()
            dd = ds.distribution(d, 0, [])
            hd = hs.distribution(logits, [])
            assert list(dd.ids) == list(hd.ids)
            assert np.allclose(dd.probs, hd.probs, rtol=1e-14, atol=0)
            assert ds.sample(d, 0, []) == hs.sample(logits, [])
        ds.close()
        d.reset()
    d.close()


@pytest.mark.timeout(900)
def test_c4_16k_context_verify_rollback_and_sampling(gpu, pair_8b):
    t_spec, d_spec = pair_8b
    P = 16384
    ctx = P + 64
    prompt = synth.seeded_ids(P, 2025, t_spec.vocab)
    ver = synth.seeded_ids(9, 33, t_spec.vocab)
    print("case c4: build and prefill 16384 tokens", flush=True)
    t = synth.build_on_device(t_spec, ctx=ctx, kv="f16")
    d = synth.build_on_device(d_spec, ctx=ctx, kv="f16")
    for i in range(0, P, 16):
        t.forward_batch(prompt[i:i + 16], logits="none")
        if i % 4096 == 0:
            print(f"c4 target prefill {i}", flush=True)
    # a 9-row verify pass (k = 8) equals nine single-token passes
    rows = t.forward_batch(ver, logits="all").copy()
    t.truncate(P)
    seq = np.stack([t.forward(x).copy() for x in ver])
    assert (_bits(rows) == _bits(seq)).all()
    print("c4: 9-row verify == 9 single passes", flush=True)
    # rollback after a verify pass: 3 rows accepted, then a continuation of 2 tokens equals the sequential one
    t.truncate(P)
    t.forward_batch(ver, logits="all")
    t.truncate(P + 3)
    cont = t.forward_batch([11, 12], logits="all").copy()
    t.truncate(P)
    for x in ver[:3]:
        t.forward(x)
    fresh = np.stack([t.forward(11).copy(), t.forward(12).copy()])
    assert (_bits(cont) == _bits(fresh)).all()
    print("c4: rollback == fresh continuation", flush=True)
    # stochastic acceptance, k = 8, temperature 0.7, top-k 40, top-p 0.9: seeded runs reproduce token for token (the
    # target keeps the prompt's cached prefix; the first run prefills the draft)
    outs = []
    for r in range(2):
        s = HipSampler(temperature=0.7, top_k=40, top_p=0.9, seed=1234)
        log, st = [], {}
        outs.append((list(generate_speculative(t, d, prompt, k=8, max_tokens=12, sample=s, stats=st, cycle_log=log)),
                     log, s.rng_state))
        s.close()
        print(f"c4: stochastic run {r}: {len(outs[-1][0])} tokens, {st['speculative']['cycles']} cycles", flush=True)
    assert outs[0] == outs[1] and len(outs[0][0]) == 12
    # every cycle consumed kk draft draws, one accept uniform per tested draft and one residual or bonus draw
    for kk, drafted, a, tok in outs[0][1]:
        assert 0 <= a <= kk <= 8 and len(drafted) == kk and 0 <= tok < t_spec.vocab
    t.close()
    d.close()


@pytest.mark.timeout(600)
def test_c5_4b_hybrid_2048_prefix_verify_state_and_rollback(gpu):
    spec = synth.qwen35_4b()
    P = 2048
    pre = synth.seeded_ids(P, 41, spec.vocab)
    ver = synth.seeded_ids(5, 42, spec.vocab)
    print("case c5: build and prefill 2048 tokens", flush=True)
    m = synth.build_on_device(spec, ctx=P + 64, kv="f16")
    for i in range(0, P, 16):
        m.forward_batch(pre[i:i + 16], logits="none")
    conv0, ssm0 = m.recurrent_state()
    m.mark_rollback()
    rows = m.forward_batch(ver, logits="all").copy()
    conv_b, ssm_b = m.recurrent_state()
    # rollback to 2 accepted tokens: snapshot restore + replay of the 2 tokens
    assert m.truncate(P + 2) == 2
    conv_r, ssm_r = m.recurrent_state()
    # the sequential path from the same state: restore the prefix state by truncating to P, then single tokens
    m.truncate(P)
    c_p, s_p = m.recurrent_state()
    assert (c_p == conv0).all() and (s_p == ssm0).all()
    seq = []
    for i, x in enumerate(ver):
        seq.append(m.forward(x).copy())
        if i == 1:
            conv_2, ssm_2 = m.recurrent_state()
    conv_s, ssm_s = m.recurrent_state()
    m.close()
    assert (_bits(rows) == _bits(np.stack(seq))).all(), "5-row verify == 5 single-token passes"
    assert (conv_b == conv_s).all() and (ssm_b == ssm_s).all(), "state after the verify == state after 5 passes"
    assert (conv_r == conv_2).all() and (ssm_r == ssm_2).all(), "rollback to 2 accepted == 2 sequential passes"
    print("c5: verify, state and rollback checks hold at a 2048-token prefix", flush=True)
