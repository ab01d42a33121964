"""GPU parity of speculative sampling: the device cycle (draft draws, accept uniforms, residual and bonus draws,
k_accept / draw_residual / draw_dist in zl_sample.hip) against the oracle's restatement of generateSpeculative
(oracle/spec.py, src/model/speculative.js:155-209) on the same GGUF files and seeds.

The tiny models' logits equal the oracle's bit for bit (test_gpu_model.py), so given the same seed every decision must
be the same: per cycle the drafted ids, the accepted count and the correction / bonus token, the emitted stream, and
the sampler's final mulberry32 state (which counts and orders every uniform consumed)."""
import numpy as np
import pytest

from oracle import oracle as O
from oracle import spec as OS
from zerollm_amd import model as Mdl
from zerollm_amd.sampler import HipSampler
from zerollm_amd.speculative import generate_speculative

pytestmark = pytest.mark.gpu

CONFIGS = {
    "T0.7-top40-p0.9": dict(temperature=0.7, top_k=40, top_p=0.9),
    "T1-top10-penalties": dict(temperature=1.0, top_k=10, top_p=0.95, repeat_penalty=1.3, repeat_last_n=16,
                                presence_penalty=-0.5, frequency_penalty=0.1),
    "T0.8-top40-minp": dict(temperature=0.8, top_k=40, top_p=1.0, min_p=0.05),
    # full candidate lists (src/sampling/sampler.js:115-118) and a top-k above the fixed lists' 256
    "T0.9-all-p0.95": dict(temperature=0.9, top_k=0, top_p=0.95),
    "T1-all-penalties-minp": dict(temperature=1.0, top_k=0, top_p=1.0, min_p=0.002, repeat_penalty=1.2, repeat_last_n=16),
    "T1.2-top300-p0.98": dict(temperature=1.2, top_k=300, top_p=0.98),
}


def _prompt(n, seed):
    r = O.Rng(seed)
    return [int(r() * 32000) for _ in range(n)]


def _run_pair(files, prompt, k, cfg, seed, max_tokens, kv="f16"):
    t = Mdl.HipModel.load(files[0], ctx=256, kv=kv)
    d = Mdl.HipModel.load(files[1], ctx=256, kv=kv)
    s = HipSampler(seed=seed, **cfg)
    log, st = [], {}
    out = list(generate_speculative(t, d, prompt, k=k, max_tokens=max_tokens, sample=s, stats=st, cycle_log=log))
    rng = s.rng_state
    limit = Mdl.verify_limit(t)
    for x in (t, d, s):
        x.close()
    return out, log, rng, st, limit


def _run_oracle(files, prompt, k, cfg, seed, max_tokens, t_limit, kv="f16"):
    t = O.OracleModel(files[0], ctx=256, kv=kv)
    d = O.OracleModel(files[1], ctx=256, kv=kv)
    s = O.Sampler(seed=seed, **cfg)
    log, st = [], {}
    out = list(OS.speculative(t, d, prompt, k=k, max_tokens=max_tokens, sample=s, stats=st, cycle_log=log,
                              t_limit=t_limit))
    return out, log, s.rng.state, st


@pytest.mark.parametrize("k", [1, 4, 8])
@pytest.mark.parametrize("seed", [1234, 99])
def test_sampled_cycles_match_oracle(gpu, close_files, k, seed):
    cfg = CONFIGS["T0.7-top40-p0.9"]
    prompt = _prompt(24, seed=11 + k)
    print(f"case sampled k={k} seed={seed}", flush=True)
    out, log, rng, st, limit = _run_pair(close_files, prompt, k, cfg, seed, 40)
    o_out, o_log, o_rng, o_st = _run_oracle(close_files, prompt, k, cfg, seed, 40, limit)
    for c, (g, w) in enumerate(zip(log, o_log)):
        assert g == w, f"cycle {c}: device {g} vs oracle {w}"
    assert log == o_log
    assert out == o_out and len(out) == 40
    assert rng == o_rng
    if k > 1:  # the accept and the reject branch both ran
        assert any(a == kk and kk > 0 for kk, _, a, _ in log) and any(a < kk for kk, _, a, _ in log)
    print(f"k={k} seed={seed}: {len(log)} cycles, accept {st['speculative']['acceptRate']:.3f}", flush=True)


@pytest.mark.parametrize("name", ["T1-top10-penalties", "T0.8-top40-minp", "T0.9-all-p0.95", "T1-all-penalties-minp",
                                  "T1.2-top300-p0.98"])
def test_sampled_cycles_match_oracle_other_samplers(gpu, close_files, name):
    """Repetition / presence / frequency penalties (the tentative tokens of a block enter the history of the later
    rows) and min-p, with the stop-token and max-token bookkeeping of the host loop."""
    cfg = CONFIGS[name]
    prompt = _prompt(20, seed=31)
    print(f"case sampler {name}", flush=True)
    out, log, rng, st, limit = _run_pair(close_files, prompt, 4, cfg, 4321, 32)
    o_out, o_log, o_rng, o_st = _run_oracle(close_files, prompt, 4, cfg, 4321, 32, limit)
    assert log == o_log
    assert out == o_out and rng == o_rng


def test_greedy_close_pair_accepts_and_equals_oracle_greedy(gpu, close_files):
    """With a draft that often agrees, greedy cycles emit several tokens; the stream is the oracle's plain greedy
    stream and the per-cycle decisions are the oracle's."""
    prompt = _prompt(32, seed=41)
    t = Mdl.HipModel.load(close_files[0], ctx=256, kv="f32")
    d = Mdl.HipModel.load(close_files[1], ctx=256, kv="f32")
    log, st = [], {}
    out = list(generate_speculative(t, d, prompt, k=4, max_tokens=48, stats=st, cycle_log=log))
    limit = Mdl.verify_limit(t)
    t.close()
    d.close()
    o_log = []
    o_out = list(OS.speculative(O.OracleModel(close_files[0], ctx=256), O.OracleModel(close_files[1], ctx=256), prompt,
                                k=4, max_tokens=48, cycle_log=o_log, t_limit=limit))
    plain = list(OS.plain(O.OracleModel(close_files[0], ctx=256), prompt, 48))
    assert out == o_out == plain
    assert log == o_log
    assert 0.1 < st["speculative"]["acceptRate"] < 0.9


def test_oracle_draft_accepts_everything_when_sampling(gpu, close_files):
    """A draft identical to the target is always accepted, at any temperature (test/spec-generate.test.js:363-380)."""
    prompt = _prompt(16, seed=51)
    t = Mdl.HipModel.load(close_files[0], ctx=256)
    d = Mdl.HipModel.load(close_files[0], ctx=256)
    s = HipSampler(temperature=0.9, top_k=20, top_p=0.9, seed=77)
    st = {}
    out = list(generate_speculative(t, d, prompt, k=4, max_tokens=21, sample=s, stats=st))
    assert len(out) == 21 and st["speculative"]["acceptRate"] == 1.0
    for x in (t, d, s):
        x.close()


@pytest.mark.parametrize("cfg", ["T0.7-top40-p0.9", "greedy"])
def test_whole_cycle_graph_equals_launch_by_launch_cycle(gpu, close_files, monkeypatch, cfg):
    """A cycle captured as two graphs (draft phase, verify phase) makes the decisions the launch-by-launch cycle makes
    (ZEROLLM_CYCLE_GRAPH=0): the same drafts, accept counts, tokens and final random state, over cycles whose draft
    feed is one token (after a rejection) or two (after a full acceptance)."""
    prompt = _prompt(20, 5)
    c = {} if cfg == "greedy" else CONFIGS[cfg]
    runs = []
    for mode in ("1", "0"):
        monkeypatch.setenv("ZEROLLM_CYCLE_GRAPH", mode)
        print(f"case whole-cycle graph {cfg} mode {mode}", flush=True)
        if cfg == "greedy":
            t = Mdl.HipModel.load(close_files[0], ctx=256, kv="f16")
            d = Mdl.HipModel.load(close_files[1], ctx=256, kv="f16")
            log, st = [], {}
            out = list(generate_speculative(t, d, prompt, k=4, max_tokens=40, stats=st, cycle_log=log))
            runs.append((out, log))
            t.close()
            d.close()
        else:
            out, log, rng, st, _ = _run_pair(close_files, prompt, 4, c, 77, 40)
            runs.append((out, log, rng))
    assert runs[0] == runs[1]
    log = runs[0][1]
    assert any(a == kk for kk, _, a, _ in log) and any(a < kk for kk, _, a, _ in log), \
        "the run has cycles after a full acceptance (two fed tokens) and after a rejection (one)"


def test_freeing_a_model_drops_its_cycle_graphs(gpu, close_files):
    """The whole-cycle graphs a sampler caches capture the models' buffers: freeing either model drops the entries
    that captured it, and a new pair starts its own."""
    import ctypes as C

    from zerollm_amd._lib import call

    def cached(s):
        n = C.c_int()
        call("zl_sampler_cycle_graphs", s._h, C.byref(n))
        return n.value

    prompt = _prompt(20, 5)
    s = HipSampler(argmax=True)
    for rnd in range(2):
        print(f"case cycle graph cache pair {rnd}", flush=True)
        t = Mdl.HipModel.load(close_files[0], ctx=256, kv="f16")
        d = Mdl.HipModel.load(close_files[1], ctx=256, kv="f16")
        out = list(generate_speculative(t, d, prompt, k=4, max_tokens=12, sample=s))
        assert len(out) == 12
        assert cached(s) > 0
        d.close()
        assert cached(s) == 0, "the draft's graphs are gone"
        t.close()
    s.close()
