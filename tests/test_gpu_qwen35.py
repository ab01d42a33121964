"""GPU parity of the qwen35 hybrid (Gated DeltaNet + gated attention) path on tiny models: logits and recurrent state
against the oracle (zerollm's Qwen35Model restated), batched = sequential, the checkpoint policy, truncate (snapshot
restore + replay) to every position = a fresh run, and hybrid speculative decoding = plain greedy decoding
(test/qwen35.test.js:158-244, test/qwen35-pool.test.js:209-351)."""
import numpy as np
import pytest

from oracle import oracle as O
from zerollm_amd import synth
from zerollm_amd.generate import generate
from zerollm_amd.speculative import generate_speculative

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3
IM = 1  # boundary token of these tests (a chat-turn start)


def prompt(n, seed=1, vocab=2048):
    r = O.Rng(seed)
    return [int(r() * vocab) for _ in range(n)]


_arrays = {}


def arrays_of(spec):
    if spec.name + str(spec.tensors[0].seed) not in _arrays:
        _arrays[spec.name + str(spec.tensors[0].seed)] = {t.name: synth.tensor_bytes(t) for t in spec.tensors}
    return _arrays[spec.name + str(spec.tensors[0].seed)]


def oracle(spec, ctx=128, kv="f32", **kw):
    return O.OracleModel(O.ArraySource(spec, arrays_of(spec)), ctx=ctx, kv=kv, **kw)


def check_close(got, want, what):
    d = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))
    assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS, (what, d.max(), d.mean())
    return d


@pytest.mark.parametrize("quant,kv", [("q8_0", "f32"), ("q4_k_m", "f16"), ("f32", "f32")])
def test_logits_and_state_match_oracle(gpu, quant, kv):
    spec = synth.tiny_qwen35(seed=21, quant=quant)
    toks = prompt(24, seed=5)
    ref = oracle(spec, kv=kv)
    want = np.stack([ref.forward(t) for t in toks])
    print(f"case qwen35 {quant} kv={kv}", flush=True)
    m = synth.build_on_device(spec, ctx=128, kv=kv)
    got = np.stack([m.forward(t).copy() for t in toks])
    d = check_close(got, want, quant)
    exact = np.mean(got.view(np.uint32) == want.view(np.uint32))
    print(f"{quant} kv={kv}: max-abs {d.max():.3g}, mean-abs {d.mean():.3g}, bit-exact {exact:.4f}")
    assert (got.argmax(1) == want.argmax(1)).all()
    # f64 sums in another order than the oracle's: the f32 logits differ only at rare rounding boundaries
    assert exact >= 0.999 and d.max() <= 1e-6 * np.abs(want).max(), (exact, d.max())
    conv, ssm = m.recurrent_state()
    rconv, rssm = ref.state()
    np.testing.assert_allclose(conv, rconv, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(ssm, rssm, rtol=1e-4, atol=1e-5)
    m.close()
    ref.close()


@pytest.mark.parametrize("form", ["matrix-core", "per-head"])
def test_gated_attention_forms_give_the_same_bits(gpu, monkeypatch, form):
    """The gated attention's weighted sum on the matrix cores for every pass, single tokens included
    (ZEROLLM_ATTN_MMAV_B=1: the form 256-dimension heads take beyond ~29,900 positions, where the slice form's softmax
    row leaves LDS), and the per-head and grouped forms of long contexts (ZEROLLM_ATTN_HEAD_CTX=0,
    ZEROLLM_ATTN_HEAD1_CTX=0) give the default forms' logits bit for bit (the slice form of single-token passes, the
    lane chains of several-token passes), over single-token and 5-token passes."""
    spec = synth.tiny_qwen35(seed=21, quant="q8_0")
    toks = prompt(40, seed=6)

    def run():
        m = synth.build_on_device(spec, ctx=128, kv="f16")
        a = np.stack([m.forward(t).copy() for t in toks[:30]])
        b = m.forward_batch(toks[30:35], logits="all").copy()
        c = np.stack([m.forward(t).copy() for t in toks[35:]])
        m.close()
        return np.concatenate([a, b, c])

    print(f"case gated attention form {form}", flush=True)
    want = run()
    if form == "matrix-core":
        monkeypatch.setenv("ZEROLLM_ATTN_MMAV_B", "1")
    else:
        monkeypatch.setenv("ZEROLLM_ATTN_HEAD_CTX", "0")
        monkeypatch.setenv("ZEROLLM_ATTN_HEAD1_CTX", "0")
    got = run()
    assert (got.view(np.uint32) == want.view(np.uint32)).all()


@pytest.mark.parametrize("d_state", [32, 128])
def test_deltanet_head_sizes_match_oracle(gpu, d_state):
    """DeltaNet heads of 32 values (one workgroup per head: no exchange among workgroups) and of 128 (four workgroups
    per head, the gated norm by the last to arrive): single-token logits and state against the oracle, and a 5-token
    pass equal to single-token passes bit for bit."""
    from zerollm_amd import gguf
    spec = synth.build_qwen35_spec(256, 2, 4, 2, 64, 32, 512, 2048, 4096, synth.qwen35_types(gguf.Q8_0), 23, interval=2,
                                   d_state=d_state, n_group=2, dt_rank=4, name=f"qwen35-dstate{d_state}")
    toks = prompt(12, seed=7)
    print(f"case deltanet d_state={d_state}", flush=True)
    ref = oracle(spec)
    want = np.stack([ref.forward(t) for t in toks])
    m = synth.build_on_device(spec, ctx=64)
    got = np.stack([m.forward(t).copy() for t in toks])
    check_close(got, want, f"d_state {d_state}")
    assert (got.argmax(1) == want.argmax(1)).all()
    assert np.mean(got.view(np.uint32) == want.view(np.uint32)) >= 0.999
    conv, ssm = m.recurrent_state()
    rconv, rssm = ref.state()
    np.testing.assert_allclose(conv, rconv, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(ssm, rssm, rtol=1e-4, atol=1e-5)
    b = synth.build_on_device(spec, ctx=64)
    for t in toks[:7]:
        b.forward(t)
    rows = b.forward_batch(toks[7:], logits="all").copy()
    assert np.array_equal(rows.view(np.uint32), got[7:].view(np.uint32))
    bconv, bssm = b.recurrent_state()
    assert np.array_equal(bconv, conv) and np.array_equal(bssm, ssm)
    for x in (m, b, ref):
        x.close()


def test_verify_width_batch_over_prefix_equals_sequential_and_oracle(gpu):
    """A 5-token verify pass (logits for every row) after a prefix: the rows equal five single-token passes bit for bit,
    and the oracle within the contract."""
    spec = synth.tiny_qwen35(seed=22, quant="q4_k_m")
    pre, ver = prompt(40, seed=6), prompt(5, seed=7)
    a = synth.build_on_device(spec, ctx=128, kv="f16")
    for i in range(0, len(pre), 16):
        a.forward_batch(pre[i:i + 16], logits="none")
    rows = a.forward_batch(ver, logits="all").copy()
    b = synth.build_on_device(spec, ctx=128, kv="f16")
    for t in pre:
        b.forward(t, logits=False)
    seq = np.stack([b.forward(t).copy() for t in ver])
    assert (rows.view(np.uint32) == seq.view(np.uint32)).all()
    sa, sb = a.recurrent_state(), b.recurrent_state()
    assert (sa[0] == sb[0]).all() and (sa[1] == sb[1]).all()
    ref = oracle(spec, kv="f16")
    for t in pre:
        ref.forward(t, logits=False)
    want = np.stack([ref.forward(t) for t in ver])
    check_close(rows, want, "verify rows")
    a.close()
    b.close()


def test_checkpoint_policy_matches_oracle(gpu):
    spec = synth.tiny_qwen35(seed=2)
    seq = [IM, 4, 5, IM, 6, 7, 8]
    for max_batch in (16, 2):
        m = synth.build_on_device(spec, ctx=64, max_batch=max_batch, boundary_ids=[IM])
        # how generate() feeds a prompt: logits only for the last token, in chunks of max_batch
        for i in range(0, len(seq), max_batch):
            chunk = seq[i:i + max_batch]
            m.forward_batch(chunk, logits="last" if i + max_batch >= len(seq) else "none")
        assert m.checkpoint_positions == [3, 6]
        assert m.truncate_plan(5) == (3, 2) and m.truncate_plan(6) == (6, 0) and m.truncate_plan(2) == (0, 2)
        assert m.truncate(5) == 2
        assert m.checkpoint_positions == [3, 5]
        m.reset()
        assert m.checkpoint_positions == [] and m.pos == 0
        m.close()
    small = synth.build_on_device(spec, ctx=64, max_checkpoints=2, boundary_ids=[IM])
    small.forward_batch([IM, 4, IM, 5, IM, 6, 7], logits="last")
    assert small.checkpoint_positions == [4, 6]
    small.close()


def test_truncate_to_every_position_equals_fresh_run(gpu):
    spec = synth.tiny_qwen35(seed=9)
    seq = [IM, 70, 5, 200, IM, 9, 255, 1, 17, 3, 33]
    fresh = synth.build_on_device(spec, ctx=64)
    want = [fresh.forward(t).copy() for t in seq]
    fresh.close()
    for opts in ({}, {"max_checkpoints": 0}, {"max_checkpoints": 1}, {"checkpoint_every": 3, "max_checkpoints": 2}):
        print(f"case truncate {opts}", flush=True)
        m = synth.build_on_device(spec, ctx=64, boundary_ids=[IM], **opts)
        for t in seq:
            m.forward(t)
        for cut in range(len(seq), -1, -1):
            frm, replay = m.truncate_plan(cut)
            got = m.truncate(cut)
            assert got == (0 if cut == len(seq) else replay)
            assert m.pos == cut and m.tokens == seq[:cut]
            for i in range(cut, len(seq)):
                assert (m.forward(seq[i]).view(np.uint32) == want[i].view(np.uint32)).all(), (opts, cut, i)
        m.close()


def test_rollback_slot_makes_partial_acceptance_a_short_replay(gpu):
    """markRollback before a verify pass, then truncate into it: the replay covers only the accepted tokens, and the
    result equals a fresh run."""
    spec = synth.tiny_qwen35(seed=13, quant="q4_k_m")
    pre, ver = prompt(12, seed=8), prompt(5, seed=9)
    m = synth.build_on_device(spec, ctx=64, kv="f16")
    m.forward_batch(pre, logits="last")
    m.mark_rollback()
    m.forward_batch(ver, logits="all")
    assert m.truncate_plan(len(pre) + 2) == (len(pre), 2)
    assert m.truncate(len(pre) + 2) == 2
    nxt = m.forward(77).copy()
    f = synth.build_on_device(spec, ctx=64, kv="f16")
    f.forward_batch(pre + ver[:2], logits="none")
    assert (f.forward(77).view(np.uint32) == nxt.view(np.uint32)).all()
    conv, ssm = m.recurrent_state()
    fc, fs = f.recurrent_state()
    assert (conv == fc).all() and (ssm == fs).all()
    m.close()
    f.close()


def test_hybrid_speculative_greedy_equals_plain_greedy(gpu):
    """test/qwen35-pool.test.js:323-349: hybrid target and hybrid draft, rollback by snapshot + replay."""
    tspec = synth.tiny_qwen35(seed=51)
    dspec = synth.tiny_qwen35(seed=52, n_layer=2, interval=2)
    p = [3, 70, 5, 200, 12, 9]
    plain = synth.build_on_device(tspec, ctx=96)
    want = list(generate(plain, p, max_tokens=24))
    T = synth.build_on_device(tspec, ctx=96, max_batch=8)
    D = synth.build_on_device(dspec, ctx=96)
    for k in (1, 3, 5):
        print(f"case hybrid speculative k={k}", flush=True)
        st = {}
        got = list(generate_speculative(T, D, p, k=k, max_tokens=24, stats=st))
        assert got == want, k
        assert st["speculative"]["cycles"] > 0
    p2 = p + want[:5] + [77]
    plain.truncate(0)
    want2 = list(generate(plain, p2, max_tokens=12))
    got2 = list(generate_speculative(T, D, p2, k=3, max_tokens=12))
    assert got2 == want2
    # a draft equal to the target is always accepted
    D2 = synth.build_on_device(tspec, ctx=96)
    st = {}
    got3 = list(generate_speculative(T, D2, p, k=4, max_tokens=16, stats=st))
    assert got3 == want[:16] and st["speculative"]["acceptRate"] == 1.0
    for x in (plain, T, D, D2):
        x.close()


def test_4b_shapes_verify_window_matches_oracle(gpu):
    """The Qwen3.5-4B-shaped Q4_K_M hybrid (the real file's tensor set and types): a short prefix, markRollback, a 5-token
    verify pass with logits for every row, then rollback to 2 accepted tokens; logits rows and the recurrent state after
    the rollback against the oracle running the same tokens one at a time."""
    spec = synth.qwen35_4b()
    pre, ver = prompt(3, seed=11, vocab=spec.vocab), prompt(5, seed=12, vocab=spec.vocab)
    print("case qwen35-4b verify window", flush=True)
    m = synth.build_on_device(spec, ctx=64, kv="f16")
    m.forward_batch(pre, logits="last")
    m.mark_rollback()
    rows = m.forward_batch(ver, logits="all").copy()
    assert m.truncate(len(pre) + 2) == 2
    conv, ssm = m.recurrent_state()
    m.close()
    arrays = {t.name: synth.tensor_bytes(t, use_device=True) for t in spec.tensors}
    O.set_threads(16)
    ref = O.OracleModel(O.ArraySource(spec, arrays), ctx=64, kv="f16", threads=16)
    for t in pre:
        ref.forward(t, logits=False)
    want = []
    for i, t in enumerate(ver):
        want.append(ref.forward(t))
        if i == 1:
            rconv, rssm = (x.copy() for x in ref.state())
    d = check_close(np.stack(rows), np.stack(want), "4b verify rows")
    print(f"qwen35-4b verify rows: max-abs {d.max():.3g}, mean-abs {d.mean():.3g}, bit-exact {np.mean(rows == np.stack(want)):.4f}")
    np.testing.assert_allclose(conv, rconv, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(ssm, rssm, rtol=1e-4, atol=1e-5)
    ref.close()


def test_verify_window_capture_equals_restore_and_replay(gpu, monkeypatch):
    """A verify pass (every row's logits) captures the recurrent state after each of its tokens, and a rollback into
    the window copies the captured state instead of restoring the snapshot and replaying the accepted tokens
    (src/compute/pool.js:278-294). Against the same model with capture off: the same replay count, checkpoint
    positions, recurrent state and next-token logits, bit for bit, for every accepted count."""
    spec = synth.tiny_qwen35(seed=23)
    pre, ver = prompt(20, seed=31), prompt(5, seed=32)
    models = {}
    for mode, env in (("capture", "1"), ("replay", "0")):
        monkeypatch.setenv("ZEROLLM_STATE_CAPTURE", env)
        models[mode] = synth.build_on_device(spec, ctx=96, kv="f16")
        models[mode].forward_batch(pre[:16], logits="none")
        models[mode].forward_batch(pre[16:], logits="last")
    for a in range(6):
        print(f"case capture a={a}", flush=True)
        out = {}
        for mode, m in models.items():
            m.truncate(len(pre))
            m.mark_rollback()
            m.forward_batch(ver, logits="all")
            replayed = m.truncate(len(pre) + a)
            conv, ssm = m.recurrent_state()
            nxt = m.forward(7).copy()
            out[mode] = (replayed, list(m.checkpoint_positions), conv, ssm, nxt)
        c, r = out["capture"], out["replay"]
        assert c[0] == r[0] and c[1] == r[1], (a, c[:2], r[:2])
        assert (c[2] == r[2]).all() and (c[3] == r[3]).all()
        assert (c[4].view(np.uint32) == r[4].view(np.uint32)).all()
    for m in models.values():
        m.close()
