"""GPU parity of the whole path on the tiny qwen3 pair (Q8_0, d 512, 4 / 2 layers, vocab 32000): logits against the
oracle (zerollm's RefModel restated), batched = sequential, KV rollback, device sampling, and speculative decoding."""
import numpy as np
import pytest

from oracle import oracle as O
from zerollm_amd import model as Mdl
from zerollm_amd.generate import generate
from zerollm_amd.sampler import HipSampler
from zerollm_amd.speculative import generate_speculative

pytestmark = pytest.mark.gpu

# logits tolerance of the parity contract (fp32 results; the path reproduces the reference's rounding points, so the
# observed differences are far below it)
MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def prompt(n, seed=1, vocab=32000):
    r = O.Rng(seed)
    return [int(r() * vocab) for _ in range(n)]


@pytest.mark.parametrize("kv", ["f32", "f16"])
def test_logits_match_oracle(gpu, tiny_files, kv):
    toks = prompt(40)
    ref = O.OracleModel(tiny_files[0], ctx=128, kv=kv)
    want = np.stack([ref.forward(t) for t in toks])
    m = Mdl.HipModel.load(tiny_files[0], ctx=128, kv=kv)
    got = np.stack([m.forward(t).copy() for t in toks])
    m.close()
    diff = np.abs(got - want)
    assert diff.max() <= MAX_ABS and diff.mean() <= MEAN_ABS, (diff.max(), diff.mean())
    exact = np.mean(got.view(np.uint32) == want.view(np.uint32))
    print(f"kv={kv}: max-abs {diff.max():.3g}, mean-abs {diff.mean():.3g}, bit-exact {exact:.4f}")
    assert (got.argmax(1) == want.argmax(1)).all()
    # the path reproduces the reference's rounding points: f64 sums in another order differ only where a sum falls
    # within ~1e-16 relative of an f32 rounding boundary
    assert exact >= 0.999 and diff.max() <= 1e-6 * np.abs(want).max(), (exact, diff.max())


@pytest.mark.parametrize("n_embd", [1024, 832])
def test_logits_match_oracle_other_widths(gpu, tmp_path, n_embd):
    """Model widths whose single-token GEMVs take the fused RMSNorm prologue with 8 and more values per thread
    (1024: the 0.6B draft's width) and a width that is not a multiple of 256 (832: clamped loads), bit-exact."""
    from zerollm_amd import synth

    t, _ = synth.tiny_pair(n_embd=n_embd)
    path = str(tmp_path / f"w{n_embd}.gguf")
    synth.write_gguf(path, t)
    toks = prompt(12, seed=13)
    ref = O.OracleModel(path, ctx=64)
    want = np.stack([ref.forward(x) for x in toks])
    print(f"case width {n_embd}", flush=True)
    m = Mdl.HipModel.load(path, ctx=64)
    got = np.stack([m.forward(x).copy() for x in toks])
    m.close()
    exact = np.mean(got.view(np.uint32) == want.view(np.uint32))
    print(f"width {n_embd}: bit-exact {exact:.5f}, max-abs {np.abs(got - want).max():.3g}")
    assert exact >= 0.999 and np.abs(got - want).max() <= 1e-6 * np.abs(want).max()


def test_forward_batch_all_equals_sequential(gpu, tiny_files):
    toks = prompt(24, seed=2)
    a = Mdl.HipModel.load(tiny_files[0], ctx=128, kv="f16")
    seq = np.stack([a.forward(t).copy() for t in toks])
    b = Mdl.HipModel.load(tiny_files[0], ctx=128, kv="f16")
    rows = []
    for chunk in (toks[:5], toks[5:6], toks[6:15], toks[15:24]):
        rows.append(b.forward_batch(chunk, logits="all").copy())
    bat = np.concatenate(rows)
    assert (bat.view(np.uint32) == seq.view(np.uint32)).all()
    last = b.forward_batch([toks[0], toks[1]], logits="last").copy()
    assert b.pos == 26
    a.forward(toks[0])
    assert (last.view(np.uint32) == a.forward(toks[1]).view(np.uint32)).all()
    a.close()
    b.close()


@pytest.mark.parametrize("kv", ["f16", "f32"])
def test_matrix_core_scores_equal_the_lane_chains(gpu, tiny_files, monkeypatch, kv):
    """Passes of several tokens with their score dots and weighted sums on the matrix cores (k_attn_prep +
    k_attn_scores_mm, k_attn_softmax_rows + k_attn_av_mm; forced for every pass of 2 tokens or more by
    ZEROLLM_ATTN_MM_B=2) give the rows of single-token passes (k_attn_scores, k_attn_av) bit for bit, over a prefix long
    enough for several position chunks, and match the oracle."""
    monkeypatch.setenv("ZEROLLM_ATTN_MM_B", "2")
    toks = prompt(600, seed=23)
    print(f"case matrix-core scores kv {kv}", flush=True)
    a = Mdl.HipModel.load(tiny_files[0], ctx=640, kv=kv)
    b = Mdl.HipModel.load(tiny_files[0], ctx=640, kv=kv, max_batch=64)
    for i in range(0, 590, 64):
        b.forward_batch(toks[i:min(i + 64, 590)], logits="none")
    for t in toks[:590]:
        a.forward(t, logits=False)
    seq = np.stack([a.forward(t).copy() for t in toks[590:]])
    bat = b.forward_batch(toks[590:], logits="all").copy()
    assert (bat.view(np.uint32) == seq.view(np.uint32)).all()
    a.close()
    b.close()
    ref = O.OracleModel(tiny_files[0], ctx=640, kv=kv)
    for t in toks[:596]:
        ref.forward(t, logits=False)
    want = np.stack([ref.forward(t) for t in toks[596:]])
    got = bat[6:]
    exact = np.mean(got.view(np.uint32) == want.view(np.uint32))
    assert exact >= 0.999 and np.abs(got - want).max() <= 1e-6 * np.abs(want).max(), exact


def test_rollback_equals_fresh_run(gpu, tiny_files):
    """50 random accept/reject cycles leave the same state as a fresh sequential run (test/spec-logits.test.js:97-139)."""
    rng = np.random.default_rng(4)
    m = Mdl.HipModel.load(tiny_files[0], ctx=512, kv="f16")
    seq = prompt(8, seed=3)
    m.forward_batch(seq, logits=False)
    for _ in range(50):
        k = int(rng.integers(1, 6))
        cand = [int(x) for x in rng.integers(0, 32000, k)]
        m.forward_batch(cand, logits="all")
        keep = int(rng.integers(0, k + 1))
        seq += cand[:keep]
        m.truncate(len(seq))
    fresh = Mdl.HipModel.load(tiny_files[0], ctx=512, kv="f16")
    for i in range(0, len(seq) - 1, 16):
        fresh.forward_batch(seq[i:min(i + 16, len(seq) - 1)], logits=False)
    a = fresh.forward(seq[-1]).copy()
    m.truncate(len(seq) - 1)
    b = m.forward(seq[-1]).copy()
    assert (a.view(np.uint32) == b.view(np.uint32)).all()
    m.close()
    fresh.close()


def test_errors_carry_reference_messages(gpu, tiny_files):
    m = Mdl.HipModel.load(tiny_files[0], ctx=8, max_batch=4, logits_batch=2)
    with pytest.raises(Exception, match="out of range"):
        m.forward(32000)
    with pytest.raises(Exception, match=r"batch of 5 tokens \(max 4\)"):
        m.forward_batch([1, 2, 3, 4, 5])
    with pytest.raises(Exception, match="logitsBatch"):
        m.forward_batch([1, 2, 3], logits="all")
    m.forward_batch([1, 2, 3, 4], logits=False)
    m.forward_batch([1, 2, 3, 4], logits=False)
    with pytest.raises(Exception, match=r"context full \(8 tokens\)"):
        m.forward(1)
    m.close()
    m.close()
    with pytest.raises(Exception, match="model is closed"):
        m.forward(1)


def test_device_sampler_matches_oracle(gpu, tiny_files):
    m = Mdl.HipModel.load(tiny_files[0], ctx=64)
    toks = prompt(6, seed=8)
    for cfg in [dict(temperature=0.7, top_k=40, top_p=0.9), dict(temperature=1.0, top_k=5, top_p=1.0, min_p=0.05),
                dict(temperature=0.8, top_k=40, top_p=0.95, repeat_penalty=1.3, presence_penalty=0.2, frequency_penalty=0.1),
                dict(temperature=0),
                # full candidate lists (topK 0: every id sorted, src/sampling/sampler.js:115-118) and topK above 256
                dict(temperature=0.7, top_k=0, top_p=0.9), dict(temperature=1.5, top_k=0, top_p=1.0),
                dict(temperature=1.0, top_k=0, top_p=0.95, min_p=0.001, repeat_penalty=1.3, presence_penalty=0.2),
                dict(temperature=1.0, top_k=1000, top_p=1.0)]:
        ds = HipSampler(seed=77, **cfg)
        hs = O.Sampler(seed=77, **cfg)
        for t in toks:
            logits = m.forward(t).copy()
            hist = toks[:3]
            dd = ds.distribution(m, 0, hist)
            hd = hs.distribution(logits, hist)
            assert list(dd.ids) == list(hd.ids)
            assert np.allclose(dd.probs, hd.probs, rtol=1e-14, atol=0)
            assert dd.greedy == hd.greedy
            assert ds.sample(m, 0, hist) == hs.sample(logits, hist)
        m.reset()
    m.close()


def test_device_sampler_ties_match_oracle(gpu, tiny_files, tmp_path):
    """Logit ties at the k-th value: which tied ids stay is decided by the reference's heap history (topKSelect,
    src/sampling/sampler.js:21-43), and a full list keeps equal logits in id order (src/sampling/sampler.js:115-118).
    An output head whose rows come in equal pairs makes every logit appear twice, so an odd top-k always cuts a pair:
    the fixed lists' heap fallback (top_k 41), the full lists' heap replay (top_k 301) and the sort's tie order
    (top_k 0) all run."""
    import shutil
    from zerollm_amd import gguf as G
    path = str(tmp_path / "paired_head.gguf")
    shutil.copy(tiny_files[0], path)
    t = G.read_gguf(path).require_tensor("output.weight")
    rb, rows = G.row_size(t.type, t.dims[0]), t.dims[1]
    with open(path, "r+b") as f:
        f.seek(t.abs_offset)
        raw = bytearray(f.read(rb * rows))
        for r in range(1, rows, 2):
            raw[r * rb:(r + 1) * rb] = raw[(r - 1) * rb:r * rb]
        f.seek(t.abs_offset)
        f.write(raw)
    m = Mdl.HipModel.load(path, ctx=64)
    toks = prompt(4, seed=9)
    for cfg in [dict(temperature=0.8, top_k=41, top_p=1.0), dict(temperature=0.8, top_k=301, top_p=1.0),
                dict(temperature=0.9, top_k=0, top_p=0.9)]:
        ds = HipSampler(seed=5, **cfg)
        hs = O.Sampler(seed=5, **cfg)
        for tk in toks:
            logits = m.forward(tk).copy()
            assert np.array_equal(logits[0::2], logits[1::2])
            dd = ds.distribution(m, 0, [])
            hd = hs.distribution(logits, [])
            assert list(dd.ids) == list(hd.ids)
            assert np.allclose(dd.probs, hd.probs, rtol=1e-14, atol=0)
            assert ds.sample(m, 0, []) == hs.sample(logits, [])
        ds.close()
        m.reset()
    m.close()


def test_device_sampler_all_equal_logits_match_oracle(gpu, tiny_files, tmp_path):
    """Every logit equal (an output head of identical rows): each 2048-logit block of the two-stage selection then holds
    more ties at its k-th value than its candidate list, so the row is selected over the whole vocabulary, and the
    reference's heap keeps the first k ids it met (topKSelect, src/sampling/sampler.js:21-43)."""
    import shutil
    from zerollm_amd import gguf as G
    path = str(tmp_path / "flat_head.gguf")
    shutil.copy(tiny_files[0], path)
    t = G.read_gguf(path).require_tensor("output.weight")
    rb, rows = G.row_size(t.type, t.dims[0]), t.dims[1]
    with open(path, "r+b") as f:
        f.seek(t.abs_offset)
        row0 = f.read(rb)
        f.seek(t.abs_offset)
        f.write(row0 * rows)
    m = Mdl.HipModel.load(path, ctx=64)
    for cfg in [dict(temperature=0.8, top_k=40, top_p=1.0), dict(temperature=1.0, top_k=5, top_p=0.9)]:
        ds = HipSampler(seed=3, **cfg)
        hs = O.Sampler(seed=3, **cfg)
        for tk in prompt(2, seed=4):
            logits = m.forward(tk).copy()
            assert np.all(logits == logits[0])
            dd = ds.distribution(m, 0, [])
            hd = hs.distribution(logits, [])
            assert list(dd.ids) == list(hd.ids)
            assert np.allclose(dd.probs, hd.probs, rtol=1e-14, atol=0)
            assert ds.sample(m, 0, []) == hs.sample(logits, [])
        ds.close()
        m.reset()
    m.close()


@pytest.mark.parametrize("k", [1, 2, 4, 7])
def test_greedy_speculative_equals_plain_greedy(gpu, tiny_files, k):
    """test/spec-generate.test.js:29-59: greedy speculative output is plain greedy output."""
    p = prompt(64, seed=5)
    t = Mdl.HipModel.load(tiny_files[0], ctx=512, kv="f16")
    d = Mdl.HipModel.load(tiny_files[1], ctx=512, kv="f16")
    st = {}
    spec = list(generate_speculative(t, d, p, k=k, max_tokens=48, stats=st))
    plain_m = Mdl.HipModel.load(tiny_files[0], ctx=512, kv="f16")
    plain = list(generate(plain_m, p, max_tokens=48))
    assert spec == plain
    assert st["speculative"]["cycles"] > 0 and st["generated"] == 48
    for x in (t, d, plain_m):
        x.close()


def test_oracle_draft_accepts_everything(gpu, tiny_files):
    """A draft identical to the target is always right (test/spec-generate.test.js:29-59)."""
    p = prompt(16, seed=6)
    t = Mdl.HipModel.load(tiny_files[0], ctx=256)
    d = Mdl.HipModel.load(tiny_files[0], ctx=256)
    st = {}
    out = list(generate_speculative(t, d, p, k=4, max_tokens=21, stats=st))
    assert len(out) == 21
    assert st["speculative"]["acceptRate"] == 1.0
    t.close()
    d.close()


def test_greedy_stream_matches_oracle(gpu, tiny_files):
    """Tiny config: 64-token prompt, greedy, k=4, f32 KV; the device stream equals the oracle's plain greedy stream."""
    p = prompt(64, seed=9)
    ref = O.OracleModel(tiny_files[0], ctx=256)
    logits = None
    for tok in p:
        logits = ref.forward(tok)
    want = []
    for _ in range(32):
        nxt = int(np.argmax(logits))
        want.append(nxt)
        logits = ref.forward(nxt)
    t = Mdl.HipModel.load(tiny_files[0], ctx=256)
    d = Mdl.HipModel.load(tiny_files[1], ctx=256)
    got = list(generate_speculative(t, d, p, k=4, max_tokens=32))
    assert got == want
    t.close()
    d.close()


def test_stop_token_and_limits(gpu, tiny_files):
    p = prompt(20, seed=10)
    t = Mdl.HipModel.load(tiny_files[0], ctx=64)
    d = Mdl.HipModel.load(tiny_files[1], ctx=64)
    plain_m = Mdl.HipModel.load(tiny_files[0], ctx=64)
    plain = list(generate(plain_m, p, max_tokens=10))
    stop = plain[3]
    st = {}
    got = list(generate_speculative(t, d, p, k=4, max_tokens=10, stop_ids={stop}, stats=st))
    assert got == plain[:plain.index(stop)]
    assert st["stopReason"] == "stop"
    st = {}
    got = list(generate_speculative(t, d, p, k=4, max_tokens=200, stats=st))
    assert len(got) == 64 - 20 + 1 and st["stopReason"] == "context"
    for x in (t, d, plain_m):
        x.close()


def test_sampled_speculative_is_reproducible(gpu, tiny_files):
    p = prompt(32, seed=11)
    runs = []
    for _ in range(2):
        t = Mdl.HipModel.load(tiny_files[0], ctx=256, kv="f16")
        d = Mdl.HipModel.load(tiny_files[1], ctx=256, kv="f16")
        s = HipSampler(temperature=0.7, top_k=40, top_p=0.9, seed=1234)
        st = {}
        runs.append(list(generate_speculative(t, d, p, k=4, max_tokens=40, sample=s, stats=st)))
        t.close()
        d.close()
    assert runs[0] == runs[1]
    assert len(runs[0]) == 40


def test_long_context_attention_matches_oracle(gpu, tiny_files):
    """Attention over 1200 cached positions (f16 KV): the last rows against the oracle run token by token."""
    toks = prompt(1204, seed=17)
    ref = O.OracleModel(tiny_files[0], ctx=1300, kv="f16")
    for t in toks[:-4]:
        ref.forward(t, logits=False)
    want = np.stack([ref.forward(t) for t in toks[-4:]])
    print("case long context 1200", flush=True)
    m = Mdl.HipModel.load(tiny_files[0], ctx=1300, kv="f16")
    for i in range(0, 1200, 16):
        m.forward_batch(toks[i:i + 16], logits="none")
    got = m.forward_batch(toks[-4:], logits="all").copy()
    m.close()
    diff = np.abs(got - want)
    assert diff.max() <= MAX_ABS and diff.mean() <= MEAN_ABS, (diff.max(), diff.mean())
    assert (got.argmax(1) == want.argmax(1)).all()


@pytest.mark.parametrize("kv", ["f16", "f32"])
def test_per_head_weighted_sum_equals_slice_form_and_oracle(gpu, tiny_files, monkeypatch, kv):
    """The long-context weighted sums forced at a 1300-position context, each against the slice form (k_attn_av) and
    the oracle:
    - "grouped": ZEROLLM_ATTN_HEAD_CTX=1024 sends passes of several tokens to k_attn_softmax_rows + k_attn_av_group
      (single-token passes keep k_attn_av);
    - "head": ZEROLLM_ATTN_HEAD1_CTX=1024 in addition sends single-token passes to the per-head kernel k_attn_av_head
      (what single-token passes take beyond ~29,900 positions).
    In every form the batched rows equal the single-token passes bit for bit, and the rows equal the slice form's."""
    toks = prompt(1210, seed=19)
    ref = O.OracleModel(tiny_files[0], ctx=1300, kv=kv)
    for t in toks[:-6]:
        ref.forward(t, logits=False)
    want = np.stack([ref.forward(t) for t in toks[-6:]])
    rows = {}
    for form in ("slice", "grouped", "head"):
        if form == "grouped":
            monkeypatch.setenv("ZEROLLM_ATTN_HEAD_CTX", "1024")
        if form == "head":
            monkeypatch.setenv("ZEROLLM_ATTN_HEAD1_CTX", "1024")
        print(f"case weighted sum {form} kv {kv}", flush=True)
        m = Mdl.HipModel.load(tiny_files[0], ctx=1300, kv=kv)
        for i in range(0, 1200, 16):
            m.forward_batch(toks[i:i + 16], logits="none")
        m.forward_batch(toks[1200:1204], logits="none")
        single = np.stack([m.forward(t).copy() for t in toks[-6:]])
        m.truncate(1204)
        batched = m.forward_batch(toks[-6:], logits="all").copy()
        m.close()
        assert (single.view(np.uint32) == batched.view(np.uint32)).all(), form
        rows[form] = single
    for form in ("grouped", "head"):
        assert (rows[form].view(np.uint32) == rows["slice"].view(np.uint32)).all(), form
    exact = np.mean(rows["head"].view(np.uint32) == want.view(np.uint32))
    assert exact >= 0.999 and np.abs(rows["head"] - want).max() <= 1e-6 * np.abs(want).max(), exact


@pytest.mark.parametrize("kv", ["f16", "f32"])
def test_matrix_core_slice_form_equals_lane_chains_and_oracle(gpu, tiny_files, monkeypatch, kv):
    """The slice form's weighted sums with the chains on the matrix cores (k_attn_av_mfma: the default from 4096
    positions, forced here by ZEROLLM_ATTN_AVMF=1) and on the lanes (k_attn_av, ZEROLLM_ATTN_AVMF=0) give the same rows
    bit for bit, for single-token passes and a 6-token pass at a 1300-position context (three staged chunks), and match
    the oracle."""
    toks = prompt(1210, seed=29)
    ref = O.OracleModel(tiny_files[0], ctx=1300, kv=kv)
    for t in toks[:-6]:
        ref.forward(t, logits=False)
    want = np.stack([ref.forward(t) for t in toks[-6:]])
    rows = {}
    for form in ("mfma", "lanes"):
        monkeypatch.setenv("ZEROLLM_ATTN_AVMF", "1" if form == "mfma" else "0")
        print(f"case slice form {form} kv {kv}", flush=True)
        m = Mdl.HipModel.load(tiny_files[0], ctx=1300, kv=kv)
        for i in range(0, 1200, 16):
            m.forward_batch(toks[i:i + 16], logits="none")
        m.forward_batch(toks[1200:1204], logits="none")
        single = np.stack([m.forward(t).copy() for t in toks[-6:]])
        m.truncate(1204)
        batched = m.forward_batch(toks[-6:], logits="all").copy()
        m.close()
        assert (single.view(np.uint32) == batched.view(np.uint32)).all(), form
        rows[form] = single
    assert (rows["mfma"].view(np.uint32) == rows["lanes"].view(np.uint32)).all()
    exact = np.mean(rows["mfma"].view(np.uint32) == want.view(np.uint32))
    assert exact >= 0.999 and np.abs(rows["mfma"] - want).max() <= 1e-6 * np.abs(want).max(), exact


def test_16k_context_verify_width_9_equals_sequential_and_rolls_back(gpu, tiny_files):
    """At a 16384-token context a 9-row verify pass (k = 8) equals nine single-token passes bit for bit, and after a
    rollback to 3 accepted rows the next pass equals a fresh continuation (size-independent checks of the long-context
    configuration)."""
    from zerollm_amd import synth

    ctx = 16384 + 32
    toks = prompt(16384 + 9, seed=18)
    print("case 16k context", flush=True)
    spec, _ = synth.tiny_pair()
    spec.ctx_train = 32768  # the tiny target with a trained context that admits 16K positions
    a = synth.build_on_device(spec, ctx=ctx, kv="f16")
    assert a.ctx == ctx
    for i in range(0, 16384, 16):
        a.forward_batch(toks[i:i + 16], logits="none")
    rows = a.forward_batch(toks[16384:], logits="all").copy()
    a.truncate(16384)
    seq = np.stack([a.forward(t).copy() for t in toks[16384:]])
    assert (rows.view(np.uint32) == seq.view(np.uint32)).all()
    a.truncate(16384 + 3)
    nxt = a.forward(5).copy()
    a.truncate(16384 + 3)
    assert (a.forward(5).view(np.uint32) == nxt.view(np.uint32)).all()
    a.close()


def _check_simd_tolerance(got, want, what, min_cos=0.9999):
    """The reference's criterion for its SIMD path against the plain-JS one (test/kquant-model.test.js:33-53): every
    row within 2e-2 x its largest logit, cosine > 0.9999, and the same argmax wherever the top-2 margin is more than 3x
    the row's largest difference. The position-split weighted sum is more
    accurate than the reference's f32 chain, but a 1e-6 relative change of an attention output flips int8 activation
    codes of these random-weight models, so it cannot meet the 2e-2 / 2e-3 absolute tolerance that bit-exact paths
    meet with zero difference; the absolute differences are printed."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    diff = np.abs(got - want)
    cos = (got * want).sum(1) / np.sqrt((got * got).sum(1) * (want * want).sum(1))
    print(f"{what}: max-abs {diff.max():.3g}, mean-abs {diff.mean():.3g}, min cosine {cos.min():.7f}", flush=True)
    assert (diff.max(1) <= 2e-2 * np.abs(want).max(1)).all()
    assert cos.min() > min_cos
    top2 = np.sort(want, axis=1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 3 * diff.max(1)
    assert (got.argmax(1) == want.argmax(1))[clear].all()


def test_split_weighted_sum_matches_oracle_at_1200_positions(gpu, tiny_files, monkeypatch):
    """Contexts beyond ZEROLLM_ATTN_EXACT_CTX take the position-split weighted sum (f64 chunk sums, online-softmax
    merge): within the reference's SIMD tolerance of the oracle's f32 chain, and batched = sequential bit for bit."""
    monkeypatch.setenv("ZEROLLM_ATTN_EXACT_CTX", "1024")
    toks = prompt(1204, seed=17)
    ref = O.OracleModel(tiny_files[0], ctx=1300, kv="f16")
    for t in toks[:-4]:
        ref.forward(t, logits=False)
    want = np.stack([ref.forward(t) for t in toks[-4:]])
    print("case split weighted sum 1200", flush=True)
    m = Mdl.HipModel.load(tiny_files[0], ctx=1300, kv="f16")
    for i in range(0, 1200, 16):
        m.forward_batch(toks[i:i + 16], logits="none")
    got = m.forward_batch(toks[-4:], logits="all").copy()
    m.truncate(1200)
    seq = np.stack([m.forward(t).copy() for t in toks[-4:]])
    m.close()
    assert (got.view(np.uint32) == seq.view(np.uint32)).all()
    _check_simd_tolerance(got, want, "split vs oracle")


def test_split_weighted_sum_matches_exact_chain_at_16k(gpu, monkeypatch):
    """At 16384 positions (the long-context configuration's length) the split weighted sum against the exact f32
    chain (bit-exact with the oracle at shorter contexts) on the same model and tokens: the deviation the split path
    has at that length."""
    from zerollm_amd import synth

    ctx = 16384 + 32
    toks = prompt(16384 + 5, seed=19)
    spec, _ = synth.tiny_pair()
    spec.ctx_train = 32768
    rows = {}
    for mode, thr in (("exact", "100000"), ("split", "1024")):
        monkeypatch.setenv("ZEROLLM_ATTN_EXACT_CTX", thr)
        print(f"case 16k {mode}", flush=True)
        m = synth.build_on_device(spec, ctx=ctx, kv="f16")
        for i in range(0, 16384, 16):
            m.forward_batch(toks[i:i + 16], logits="none")
        rows[mode] = m.forward_batch(toks[16384:], logits="all").copy()
        m.close()
    # observed: max-abs 0.031, mean-abs 0.0054, min cosine 0.99985, below the reference's 0.9999: at 16K positions
    # the path does not meet the reference's SIMD bounds on this random model, which is why contexts the exact chain
    # can hold (up to ~29900 positions) use the exact chain
    _check_simd_tolerance(rows["split"], rows["exact"], "16k split vs exact", min_cos=0.9995)
