"""CPU tests that pin the oracle's qwen35 (Gated DeltaNet hybrid) path and its checkpoint policy, as zerollm's
test/qwen35.test.js does for its reference path: against an independent whole-sequence chunk-form forward
(tests/naive_qwen35.py), closed forms of the small functions, the real Qwen3.5-4B tensor list, and the rollback
invariants (truncate to any position == a fresh run, bit for bit)."""
import math
import os

import numpy as np
import pytest

from oracle import oracle as O
from oracle.checkpoints import StateCheckpoints
from zerollm_amd import gguf as G
from zerollm_amd import synth

from naive_qwen35 import naive_qwen35_logits

TOKS = [3, 70, 5, 200, 12, 9, 255, 1, 17]
FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "qwen35-4b-tensors.txt")


def arrays_of(spec):
    return {t.name: synth.tensor_bytes(t) for t in spec.tensors}


def oracle_model(spec, arrays=None, **kw):
    arrays = arrays if arrays is not None else arrays_of(spec)
    return O.OracleModel(O.ArraySource(spec, arrays), ctx=kw.pop("ctx", 64), **kw), arrays


def weight_fns(spec, arrays):
    by = {t.name: t for t in spec.tensors}

    def W(name):
        t = by[name]
        if t.type == G.F32:
            return arrays[name].view(np.float32).reshape(t.rows, t.cols).astype(np.float64)
        return O.dequant(t.type, arrays[name], t.rows, t.cols).astype(np.float64)

    def V(name):
        return arrays[name].view(np.float32).astype(np.float64)

    return W, V


# ------------------------------------------------------------------------------------------------ small functions
def test_softplus_sigmoid_closed_forms():
    assert O.lib().orc_softplus(0.0) == pytest.approx(math.log(2.0), rel=0, abs=1e-15)
    assert O.lib().orc_softplus(25.0) == 25.0                       # linear above 20 (ggml_softplus)
    assert O.lib().orc_softplus(20.0) == pytest.approx(math.log1p(math.exp(20.0)), abs=0)
    assert O.lib().orc_softplus(-40.0) == pytest.approx(math.exp(-40.0), rel=1e-12)
    assert O.lib().orc_sigmoid(0.0) == 0.5
    assert O.lib().orc_sigmoid(3.0) + O.lib().orc_sigmoid(-3.0) == pytest.approx(1.0, abs=1e-15)


def test_conv_step_is_a_sliding_dot_product_with_silu():
    rng = np.random.default_rng(1)
    C, K, T = 6, 4, 7
    w = rng.normal(size=(C, K)).astype(np.float32)
    xs = rng.normal(size=(T, C)).astype(np.float32)
    state = np.zeros(C * (K - 1), np.float32)
    for t in range(T):
        x = xs[t].copy()
        O.lib().orc_conv_step(O.p(state, O.C.c_float), O.p(w, O.C.c_float), O.p(x, O.C.c_float), O.p(x, O.C.c_float), C, K)
        win = np.zeros((K, C))
        for i in range(K):
            tt = t - (K - 1) + i
            if tt >= 0:
                win[i] = xs[tt]
        s = (w.astype(np.float64).T * win).sum(axis=0)
        np.testing.assert_allclose(x, s / (1 + np.exp(-s)), rtol=1e-6, atol=1e-7)
        # the window holds the last K-1 inputs, oldest first
        np.testing.assert_array_equal(state.reshape(C, K - 1)[:, -1], xs[t])


def test_delta_rule_matches_matrix_form():
    """S' = g S + beta k (v - g S k)^T written as matrices (S stored [dv][dk]), o = S'^T q."""
    rng = np.random.default_rng(2)
    dk, dv = 8, 6
    S = rng.normal(size=(dv, dk)).astype(np.float32)
    q, k, v = (rng.normal(size=n).astype(np.float32) for n in (dk, dk, dv))
    g, beta = 0.83, 0.4
    want_S = g * S.astype(np.float64)
    d = beta * (v - want_S @ k)
    want_S = want_S + np.outer(d, k)
    out = np.zeros(dv, np.float32)
    Sc = S.copy()
    O.lib().orc_delta_rule_head(O.p(Sc, O.C.c_float), O.p(q, O.C.c_float), O.p(k, O.C.c_float), O.p(v, O.C.c_float),
                                O.p(out, O.C.c_float), dk, dv, g, beta)
    np.testing.assert_allclose(Sc, want_S, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(out, want_S @ q, rtol=1e-5, atol=1e-6)


def test_l2norm_and_gated_rmsnorm_closed_forms():
    rng = np.random.default_rng(3)
    v = rng.normal(size=16).astype(np.float32)
    x = v.copy()
    O.lib().orc_l2norm_heads(O.p(x, O.C.c_float), 2, 8, 1e-6, 0.25)
    for h in range(2):
        seg = v[h * 8:(h + 1) * 8].astype(np.float64)
        np.testing.assert_allclose(x[h * 8:(h + 1) * 8], 0.25 * seg / np.sqrt((seg * seg).sum() + 1e-6), rtol=1e-6)
    o = v[:8].copy()
    z = rng.normal(size=8).astype(np.float32)
    w = rng.normal(size=8).astype(np.float32)
    O.lib().orc_gated_rmsnorm_head(O.p(o, O.C.c_float), O.p(z, O.C.c_float), O.p(w, O.C.c_float), 8, 1e-6)
    ov = v[:8].astype(np.float64)
    want = ov / np.sqrt((ov * ov).mean() + 1e-6) * w * (z / (1 + np.exp(-z.astype(np.float64))))
    np.testing.assert_allclose(o, want, rtol=1e-6, atol=1e-7)


# ------------------------------------------------------------------------------------------------ tensor set
def test_synthetic_4b_spec_has_the_real_file_tensor_set():
    real = {}
    with open(FIXTURE) as f:
        for line in f:
            if line.strip() and not line.startswith("#"):
                name, ty, dims = line.split(" ", 2)
                real[name] = (ty, [int(x) for x in dims.strip()[1:-1].split(",")])
    assert len(real) == 426
    spec = synth.qwen35_4b()
    mine = {t.name: t for t in spec.tensors}
    assert sorted(mine) == sorted(real)
    names = {G.Q4_K: "Q4_K", G.Q5_K: "Q5_K", G.Q6_K: "Q6_K", G.Q8_0: "Q8_0", G.F32: "F32"}
    for n, t in mine.items():
        assert t.dims == real[n][1], n
        assert names[t.type] == real[n][0], n
    # 2.73 GB of matrices per pass (the 4B file's Q4_K_M mix), the tied embedding read one row per token
    assert 2.6e9 < spec.weight_bytes < 2.9e9


# ------------------------------------------------------------------------------------------------ forward vs naive
@pytest.mark.parametrize("seed", [3, 11])
def test_forward_equals_chunk_form_naive_on_f32_weights(seed):
    spec = synth.tiny_qwen35(seed=seed, quant="f32")
    m, arrays = oracle_model(spec)
    W, V = weight_fns(spec, arrays)
    want = naive_qwen35_logits(spec, W, V, TOKS)
    for i, t in enumerate(TOKS):
        got = m.forward(t)
        scale = max(1.0, float(np.abs(want[i]).max()))
        assert np.abs(got - want[i]).max() < 1e-4 * scale, (seed, i)
        assert int(np.argmax(got)) == int(np.argmax(want[i]))
    m.close()


@pytest.mark.parametrize("quant", ["q8_0", "q4_k_m"])
def test_forward_tracks_naive_with_quantized_weights(quant):
    spec = synth.tiny_qwen35(seed=5, quant=quant)
    if quant == "q4_k_m":
        types = {t.type for t in spec.tensors}
        assert {G.Q4_K, G.Q5_K, G.Q6_K, G.Q8_0} <= types
    m, arrays = oracle_model(spec)
    W, V = weight_fns(spec, arrays)
    toks = TOKS[:6]
    want = naive_qwen35_logits(spec, W, V, toks)
    for i, t in enumerate(toks):
        got = m.forward(t).astype(np.float64)
        cos = got @ want[i] / np.sqrt((got @ got) * (want[i] @ want[i]))
        assert cos > 0.99, (quant, i, cos)
    m.close()


@pytest.mark.parametrize("decay", [(0.5, 0.7), (0.9, 0.999)])
def test_chunked_delta_rule_is_not_the_recurrence_bits(decay):
    """Why a chunked (WY) prefill of the Gated DeltaNet is not used: over 2048 tokens of a 128 x 128 head, the chunk form
    equals the exact recurrence in f64 to 1e-15, but the reference's recurrence (deltaRuleHead,
    src/compute/ref-deltanet.js:79-90) rounds the state to f32 after every decay and every write, and those roundings are
    part of its result. Measured: the chunk form's outputs carry ~1e-7 of relative deviation from the reference's and
    equal its bits in only 46 % (fast decay) / 23 % (slow decay) of elements; per-element perturbations of this kind are
    what the random-weight networks amplify through the int8 activation rounding of every later layer (the
    position-split attention sum: ~1e-6 per element became 0.028 max-abs in the logits). The GPU runs the recurrence
    itself, token by token inside each workgroup, and captures the state per position instead."""
    from tests.naive_qwen35 import chunked_gated_delta_rule

    rng = np.random.default_rng(1)
    T, D = 2048, 128

    def l2(x):
        return x / np.sqrt((x * x).sum(-1, keepdims=True) + 1e-6)

    k = l2(rng.normal(size=(T, D))).astype(np.float32)
    q = (l2(rng.normal(size=(T, D))) / np.sqrt(D)).astype(np.float32)
    v = (rng.normal(size=(T, D)) * 0.5).astype(np.float32)
    gam = rng.uniform(decay[0], decay[1], T)
    beta = 1.0 / (1.0 + np.exp(-rng.normal(size=T)))
    # the reference's recurrence: f64 arithmetic, the state stored f32 after the decay and after the write
    S = np.zeros((D, D), np.float32)
    ref = np.zeros((T, D), np.float32)
    ex = np.zeros((T, D))
    Se = np.zeros((D, D))
    for t in range(T):
        s = (S.astype(np.float64) * gam[t]).astype(np.float32)
        d = (v[t] - s.astype(np.float64) @ k[t].astype(np.float64)) * beta[t]
        S = (s.astype(np.float64) + np.outer(d, k[t].astype(np.float64))).astype(np.float32)
        ref[t] = (S.astype(np.float64) @ q[t].astype(np.float64)).astype(np.float32)
        Se = Se * gam[t]
        de = (v[t] - Se @ k[t]) * beta[t]
        Se = Se + np.outer(de, k[t])
        ex[t] = Se @ q[t]
    wy, Swy = chunked_gated_delta_rule(q, k, v, gam, beta, chunk=64)
    assert np.abs(wy - ex).max() <= 1e-12 * np.abs(ex).max() and np.abs(Swy - Se).max() <= 1e-12 * np.abs(Se).max()
    got = wy.astype(np.float32)
    rel = np.abs(got - ref).max() / np.abs(ref).max()
    same = np.mean(got.view(np.uint32) == ref.view(np.uint32))
    print(f"decay {decay}: chunk form vs the reference's recurrence: max-abs {rel:.2e} of max, bit-equal {same:.3f}")
    assert 1e-8 < rel < 1e-5 and same < 0.6


def test_prefill_without_logits_equals_token_by_token_and_state_is_deterministic():
    spec = synth.tiny_qwen35(seed=7)
    arrays = arrays_of(spec)
    a, _ = oracle_model(spec, arrays)
    b, _ = oracle_model(spec, arrays)
    for t in TOKS[:-1]:
        a.forward(t, logits=False)
    la = a.forward(TOKS[-1])
    for t in TOKS:
        lb = b.forward(t)
    np.testing.assert_array_equal(la, lb)
    sa, sb = a.state(), b.state()
    np.testing.assert_array_equal(sa[0], sb[0])
    np.testing.assert_array_equal(sa[1], sb[1])
    assert np.any(sa[0] != 0) and np.any(sa[1] != 0)
    with pytest.raises(RuntimeError, match="context full"):
        for _ in range(70):
            a.forward(1)


# ------------------------------------------------------------------------------------------------ checkpoints
IM = 1  # the boundary token of these tests (a chat-turn start, <|im_start|> in a real vocabulary)


def test_truncate_to_every_position_equals_a_fresh_run():
    spec = synth.tiny_qwen35(seed=9)
    arrays = arrays_of(spec)
    seq = [IM, 70, 5, 200, IM, 9, 255, 1, 17, 3, 33]
    fresh, _ = oracle_model(spec, arrays)
    want = [fresh.forward(t) for t in seq]
    for opts in ({}, {"max_checkpoints": 0}, {"max_checkpoints": 1}, {"checkpoint_every": 3, "max_checkpoints": 2}):
        m, _ = oracle_model(spec, arrays, boundary_ids=[IM], **opts)
        for t in seq:
            m.forward(t)
        for cut in range(len(seq), -1, -1):
            frm, replay = m.truncate_plan(cut)
            got = m.truncate(cut)
            assert got == (0 if cut == len(seq) else replay)
            assert m.pos == cut and m.tokens == seq[:cut]
            for i in range(cut, len(seq)):
                np.testing.assert_array_equal(m.forward(seq[i]), want[i], err_msg=f"{opts} cut {cut} pos {i}")
        m.close()


def test_truncate_then_different_continuation_equals_fresh_run():
    spec = synth.tiny_qwen35(seed=12, quant="f32")
    arrays = arrays_of(spec)
    m, _ = oracle_model(spec, arrays)
    for t in [3, 70, 5, 200, 12, 9]:
        m.forward(t)
    m.truncate(4)
    got = [m.forward(t) for t in [8, 99, 4]]
    f, _ = oracle_model(spec, arrays)
    want = [f.forward(t) for t in [3, 70, 5, 200, 8, 99, 4]][4:]
    for x, y in zip(got, want):
        np.testing.assert_array_equal(x, y)


def test_checkpoint_policy_known_positions():
    """test/qwen35.test.js:224-244: before a boundary token, before the last prompt token, bounded, smallest evicted."""
    spec = synth.tiny_qwen35(seed=2)
    arrays = arrays_of(spec)
    seq = [IM, 4, 5, IM, 6, 7, 8]
    m, _ = oracle_model(spec, arrays, boundary_ids=[IM])
    for i, t in enumerate(seq):
        m.forward(t, logits=i == len(seq) - 1)
    assert m.ck.positions == [3, 6]
    assert m.truncate_plan(5) == (3, 2)
    assert m.truncate_plan(6) == (6, 0)
    assert m.truncate_plan(2) == (0, 2)
    assert m.truncate(5) == 2
    assert m.ck.positions == [3, 5]
    m.reset()
    assert m.ck.positions == [] and m.pos == 0
    small, _ = oracle_model(spec, arrays, boundary_ids=[IM], max_checkpoints=2)
    seq2 = [IM, 4, IM, 5, IM, 6, 7]
    for i, t in enumerate(seq2):
        small.forward(t, logits=i == len(seq2) - 1)
    assert small.ck.positions == [4, 6]


def test_rollback_slot_plan():
    """mark() is one slot, separate from the checkpoints, skipped where a checkpoint exists (state-checkpoints.js:53-58)."""
    ck = StateCheckpoints(max_checkpoints=2)
    live = (np.zeros(3, np.float32), np.zeros(2, np.float32))
    ck.save(4, live)
    ck.mark(4, live)
    assert ck.rollback is None
    live[0][:] = 7
    ck.mark(9, live)
    assert ck.plan(11, 12) == (9, 2)
    assert ck.plan(8, 12) == (4, 4)
    ck.drop_after(8)
    assert ck.rollback is None and ck.positions == [4]
    assert ck.plan(3, 12) == (0, 3)
