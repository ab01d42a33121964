"""CPU checks that pin the oracle's speculative decoding (oracle/spec.py, restating src/model/speculative.js:100-240).

What fixes the answers here is not the oracle's own code:
- greedy speculative output equals plain greedy output (test/spec-generate.test.js:29-59), for mock models and for the
  tiny oracle pair;
- a draft identical to the target is always accepted, at any temperature (:363-380);
- as the temperature goes to 0 the sampled cycle collapses to plain greedy (every accept / residual decision is then
  forced by a point mass);
- the number of uniforms consumed equals the count the reference's order implies (kk draft draws, one accept uniform per
  tested draft, one residual or bonus draw), checked from the mulberry32 state's closed form;
- hand-built distributions whose outcome follows from the textbook rule (Leviathan et al. 2023) and the documented
  order of the uniforms (draft draws, accept tests, residual / bonus);
- a chi-square test that the emitted tokens have exactly the target's distribution, with a power check against the
  draft's (test/spec-generate.test.js:268-361).
"""
import numpy as np
import pytest

from oracle import oracle as O
from oracle import spec as S

GOLDEN = 0x6D2B79F5
INV_GOLDEN = pow(GOLDEN, -1, 1 << 32)


class MockModel:
    """A model whose logits are a pure function of the token prefix (the reference's positional-KV invariant), over a
    small vocabulary: logits[i] = scale * N(0, 1) seeded by (seed, last `window` tokens, position). A draft made with
    noise > 0 is the target's logits plus scaled independent noise, so acceptance is partial."""

    def __init__(self, vocab=12, seed=1, scale=1.5, ctx=256, noise=0.0, noise_seed=99, window=3):
        self.vocab, self.seed, self.scale, self.ctx = vocab, seed, scale, ctx
        self.noise, self.noise_seed, self.window = noise, noise_seed, window
        self.tokens = []
        self.calls = 0

    @property
    def pos(self):
        return len(self.tokens)

    def _logits(self, toks):
        key = (len(toks),) + tuple(toks[-self.window:])
        g = np.random.default_rng([self.seed, *[int(t) + 1 for t in key]])
        l = self.scale * g.standard_normal(self.vocab)
        if self.noise:
            n = np.random.default_rng([self.noise_seed, *[int(t) + 1 for t in key]])
            l = l + self.noise * n.standard_normal(self.vocab)
        return l.astype(np.float32)

    def forward(self, token, logits=True):
        if self.pos >= self.ctx:
            raise RuntimeError(f"context full ({self.ctx} tokens)")
        if not 0 <= token < self.vocab:
            raise RuntimeError(f"token id {token} out of range")
        self.tokens.append(int(token))
        self.calls += 1
        return self._logits(self.tokens) if logits else None

    def forward_again(self):
        """The logits after the current prefix (no token is added)."""
        return self._logits(self.tokens)

    def truncate(self, n):
        del self.tokens[max(0, n):]
        return 0

    def reset(self):
        self.tokens = []


def rng_calls(seed, state):
    """Number of mulberry32 draws between seed and state (each draw adds the golden constant to the state)."""
    return ((state - seed) * INV_GOLDEN) & 0xFFFFFFFF


@pytest.mark.parametrize("k", [1, 2, 4, 7])
def test_greedy_speculative_equals_plain_greedy_mock(k):
    for p in range(10):
        prompt = [(3 * p + i) % 12 for i in range(4 + p % 3)]
        t, d = MockModel(seed=5), MockModel(seed=5, noise=1.0)
        st = {}
        spec = list(S.speculative(t, d, prompt, k=k, max_tokens=30, stats=st))
        plain = list(S.plain(MockModel(seed=5), prompt, 30))
        assert spec == plain, (k, p)
        assert 0 < st["speculative"]["acceptRate"] < 1
        full = prompt + spec
        assert t.tokens == full[:len(t.tokens)] and len(t.tokens) >= len(full) - 1
        assert d.tokens == full[:len(d.tokens)]


def test_greedy_speculative_equals_plain_greedy_tiny_oracle_pair(tiny_files):
    prompt = [int(O.Rng(5)() * 32000)] + [int(x) for x in np.random.default_rng(5).integers(0, 32000, 15)]
    t = O.OracleModel(tiny_files[0], ctx=128)
    d = O.OracleModel(tiny_files[1], ctx=128)
    log = []
    spec = list(S.speculative(t, d, prompt, k=4, max_tokens=12, cycle_log=log))
    plain = list(S.plain(O.OracleModel(tiny_files[0], ctx=128), prompt, 12))
    assert spec == plain
    assert sum(len(c[1]) for c in log) > 0


def test_speculative_greedy_wrapper_continues_a_prefilled_sequence():
    prompt = [1, 2, 3, 4, 5]
    t, d = MockModel(seed=2), MockModel(seed=2, noise=0.7)
    for m in (t, d):
        for tok in prompt[:-1]:
            m.forward(tok, logits=False)
    out, cycles = S.speculative_greedy(t, d, prompt, 4, 20)
    assert out == list(S.plain(MockModel(seed=2), prompt, 20))
    assert 0 < cycles <= 20


def test_identical_draft_accepts_everything_when_sampling():
    t, d = MockModel(seed=3), MockModel(seed=3)
    s = O.Sampler(temperature=0.9, top_k=8, top_p=0.95, seed=11)
    st = {}
    out = list(S.speculative(t, d, [1, 2, 3], k=4, max_tokens=21, sample=s, stats=st))
    assert len(out) == 21
    assert st["speculative"]["acceptRate"] == 1.0
    assert st["speculative"]["acceptedHist"][4] == st["speculative"]["cycles"] - 1  # the last cycle drafts fewer


def test_vanishing_temperature_collapses_to_greedy():
    for seed in (1, 2, 3):
        t, d = MockModel(seed=seed), MockModel(seed=seed, noise=1.5)
        s = O.Sampler(temperature=1e-4, top_k=8, top_p=0.9, seed=seed)
        spec = list(S.speculative(t, d, [4, 5, 6], k=4, max_tokens=25, sample=s))
        assert spec == list(S.plain(MockModel(seed=seed), [4, 5, 6], 25))


@pytest.mark.parametrize("k", [1, 3, 4, 8])
def test_uniforms_consumed_in_the_reference_count(k):
    """Per cycle: kk draft draws, then one accept uniform per tested draft (a accepted, +1 for the rejected one), then
    exactly one residual or bonus draw (src/model/speculative.js:169-209)."""
    seed = 1000 + k
    t, d = MockModel(seed=7), MockModel(seed=7, noise=1.2)
    s = O.Sampler(temperature=0.8, top_k=10, top_p=0.95, seed=seed)
    log = []
    list(S.speculative(t, d, [1, 2], k=k, max_tokens=60, sample=s, cycle_log=log))
    want = sum(kk + a + (1 if a < kk else 0) + 1 for kk, _, a, _ in log)
    assert any(a < kk for kk, _, a, _ in log) and any(a == kk and kk > 0 for kk, _, a, _ in log)
    assert rng_calls(seed, s.rng.state) == want


class TableModel:
    """Logits fixed per position (pos -> f32 row), to build hand-computed cycles."""

    def __init__(self, rows, ctx=64):
        self.rows, self.ctx, self.tokens = rows, ctx, []

    @property
    def pos(self):
        return len(self.tokens)

    def forward(self, token, logits=True):
        self.tokens.append(int(token))
        return np.asarray(self.rows[min(len(self.tokens) - 1, len(self.rows) - 1)], np.float32) if logits else None

    def truncate(self, n):
        del self.tokens[max(0, n):]
        return 0


def test_hand_built_cycle_follows_the_documented_uniform_order():
    """One k=2 cycle over 4 tokens, temperature 1, no top-k / top-p: q = [.1,.2,.3,.4] at both draft steps, p =
    [.4,.3,.2,.1] at every target row. With the uniforms u1..u6 of mulberry32(seed): x1 = inverse-CDF(q, u1) and
    x2 = inverse-CDF(q, u2), over the candidates in descending-probability order (the sampler's order); accept x1 iff
    u3 q(x1) < p(x1); if accepted, accept x2 iff u4 q(x2) < p(x2); the first rejection draws the residual
    max(0, p - q) = [.3, .1, 0, 0] / .4 with the next uniform; if both pass, the bonus is inverse-CDF(p, u5)."""
    q = np.log(np.array([0.1, 0.2, 0.3, 0.4]))
    p = np.log(np.array([0.4, 0.3, 0.2, 0.1]))
    seen = set()
    for seed in range(40):
        u = O.Rng(seed)
        us = [u() for _ in range(6)]
        qw, pw = np.array([0.1, 0.2, 0.3, 0.4]), np.array([0.4, 0.3, 0.2, 0.1])

        def cdf(w, x):
            order = np.argsort(-w, kind="stable")
            return int(order[np.searchsorted(np.cumsum(w[order]) / np.sum(w), x, side="left")])

        x = [cdf(qw, us[0]), cdf(qw, us[1])]
        a, i, tok = 0, 2, None
        for j in range(2):
            if us[i] * qw[x[j]] < pw[x[j]]:
                a += 1
                i += 1
                continue
            i += 1
            tok = 0 if us[i] * 0.4 <= 0.3 else 1
            break
        if a == 2:
            tok = cdf(pw, us[i])
        t = TableModel([p] * 8)
        d = TableModel([q] * 8)
        s = O.Sampler(temperature=1.0, top_k=0, top_p=1.0, seed=seed)
        log = []
        list(S.speculative(t, d, [0], k=2, max_tokens=3, sample=s, cycle_log=log))
        kk, drafted, ga, gtok = log[0]
        assert (list(drafted), ga, gtok) == (x, a, tok), seed
        seen.add((a, tok is not None))
    assert {0, 1, 2} <= {a for a, _ in seen}


def _chi_square(counts, n, dist):
    """test/spec-generate.test.js:283-299: bins with expected count < 8 are pooled."""
    stat, df, pool_e, pool_o = 0.0, -1, 0.0, 0
    support = set(int(i) for i in dist.ids)
    assert all(k in support for k in counts), "a token outside the target distribution's support was produced"
    for i, tid in enumerate(dist.ids):
        e = n * dist.probs[i] / dist.total
        o = counts.get(int(tid), 0)
        if e < 8:
            pool_e += e
            pool_o += o
            continue
        stat += (o - e) ** 2 / e
        df += 1
    if pool_e >= 5:
        stat += (pool_o - pool_e) ** 2 / pool_e
        df += 1
    return stat, df


def _critical(df):
    return df + 6 * np.sqrt(2 * df) + 6


@pytest.mark.parametrize("cfg", [dict(temperature=1.0, top_k=8, top_p=0.95, repeat_penalty=1.3, repeat_last_n=16,
                                      presence_penalty=-2.0),
                                 dict(temperature=0.8, top_k=0, top_p=0.9, min_p=0.02)])
def test_sampled_output_has_the_target_distribution(cfg):
    """test/spec-generate.test.js:268-361 on mock models: tokens 1 and 2 of 3000 seeded runs against the exact target
    distributions (with the tentative token in the history), and the draft's distribution is rejected."""
    prompt = [3, 3, 3, 3]  # one repeated id, so a tentative token almost always changes the penalties
    N = 3000
    runs = []
    drafted = accepted = 0
    for i in range(N):
        t, d = MockModel(seed=21, scale=1.2), MockModel(seed=21, scale=1.2, noise=0.9)
        s = O.Sampler(seed=int(O.Rng(i + 1)() * 2 ** 32), **cfg)
        st = {}
        runs.append(list(S.speculative(t, d, prompt, k=4, max_tokens=3, sample=s, stats=st)))
        drafted += st["speculative"]["drafted"]
        accepted += st["speculative"]["accepted"]
    rate = accepted / drafted
    assert 0.05 < rate < 0.95, rate
    exact = O.Sampler(seed=1, **cfg)
    tm = MockModel(seed=21, scale=1.2)
    for tok in prompt[:-1]:
        tm.forward(tok, logits=False)
    p1 = exact.distribution(tm.forward(prompt[-1]), prompt)
    c1 = {}
    for r in runs:
        c1[r[0]] = c1.get(r[0], 0) + 1
    stat, df = _chi_square(c1, N, p1)
    assert stat < _critical(df), (stat, df)
    dm = MockModel(seed=21, scale=1.2, noise=0.9)
    for tok in prompt[:-1]:
        dm.forward(tok, logits=False)
    q1 = exact.distribution(dm.forward(prompt[-1]), prompt)
    if all(k in set(int(i) for i in q1.ids) for k in c1):
        qs, qdf = _chi_square(c1, N, q1)
        assert qs > 3 * _critical(qdf), (qs, qdf)
    ranked = sorted(c1.items(), key=lambda kv: -kv[1])
    ranked = [kv for kv in ranked if kv[1] >= 150][:3]
    assert len(ranked) >= 2
    history_effect = 0.0
    for t1, n1 in ranked:
        sub = [r for r in runs if r[0] == t1]
        tm2 = MockModel(seed=21, scale=1.2)
        for tok in prompt:
            tm2.forward(tok, logits=False)
        p2 = exact.distribution(tm2.forward(t1), prompt + [t1])
        c2 = {}
        for r in sub:
            c2[r[1]] = c2.get(r[1], 0) + 1
        stat, df = _chi_square(c2, len(sub), p2)
        assert stat < _critical(df), (t1, stat, df)
        # how far the distribution would move without the tentative token in the history (the test's power for
        # penalties, as the reference's test guards it)
        wrong = exact.distribution(tm2.forward_again(), prompt)
        pm = {int(i): p2.probs[j] / p2.total for j, i in enumerate(p2.ids)}
        wm = {int(i): wrong.probs[j] / wrong.total for j, i in enumerate(wrong.ids)}
        history_effect = max(history_effect, sum(abs(pm.get(i, 0) - wm.get(i, 0)) for i in set(pm) | set(wm)) / 2)
    if cfg.get("presence_penalty"):
        assert history_effect > 0.1, history_effect


def test_stop_max_and_context_edges():
    """test/spec-generate.test.js:98-141 on mock models: a stop token ends the stream unemitted; the context bound
    emits exactly until the window is full."""
    prompt = [1, 2, 3]
    plain = list(S.plain(MockModel(seed=4), prompt, 12))
    stop = plain[5]
    st = {}
    got = list(S.speculative(MockModel(seed=4), MockModel(seed=4, noise=0.8), prompt, k=3, max_tokens=12,
                             stop_ids={stop}, stats=st))
    assert got == plain[:plain.index(stop)] and st["stopReason"] == "stop"
    st = {}
    got = list(S.speculative(MockModel(seed=4, ctx=16), MockModel(seed=4, noise=0.8, ctx=16), prompt, k=4,
                             max_tokens=100, stats=st))
    assert len(got) == 16 - 3 + 1 and st["stopReason"] == "context"
    assert got == list(S.plain(MockModel(seed=4, ctx=16), prompt, 100))
