"""CPU tests that pin the oracle (oracle/zl_oracle.c) against zerollm's own golden vectors and known answers, and
against what the mathematics fixes (brute force, closed forms, invariants)."""
import base64
import json
import math
import os

import numpy as np
import pytest

from oracle import oracle as O
from zerollm_amd import gguf as G

GOLD = os.path.join(os.path.dirname(__file__), "golden", "quant-vectors.json")
TYPES = {"Q5_0": G.Q5_0, "Q4_K": G.Q4_K, "Q5_K": G.Q5_K, "Q6_K": G.Q6_K}


def golden():
    with open(GOLD) as f:
        return json.load(f)


# ------------------------------------------------------------------------------------------------ f16 (test/f16.test.js:5-26)
def test_f16_known_encodings():
    assert O.f32_to_f16(1.0) == 0x3C00
    assert O.f32_to_f16(-2.0) == 0xC000
    assert O.f32_to_f16(65504.0) == 0x7BFF
    assert O.f32_to_f16(65520.0) == 0x7C00
    assert O.f32_to_f16(0.0) == 0
    assert O.f32_to_f16(2.0 ** -24) == 1
    assert O.f32_to_f16(2.0 ** -25) == 0
    assert O.f32_to_f16(1.5 * 2.0 ** -24) == 2
    assert O.f32_to_f16(float("inf")) == 0x7C00
    assert O.f32_to_f16(float("nan")) & 0x7C00 == 0x7C00


def test_f16_exhaustive_round_trip_and_numpy_agreement():
    h = np.arange(65536, dtype=np.uint16)
    finite = ((h >> 10) & 0x1F) != 0x1F
    ref = h.view(np.float16).astype(np.float32)
    for v in h[finite][::7]:
        f = O.f16_to_f32(int(v))
        assert f == ref[v] or (math.isnan(f) and math.isnan(ref[v]))
        assert O.f32_to_f16(f) == int(v)
    # RNE against numpy's independent f32 -> f16 conversion on random and halfway values
    rng = np.random.default_rng(5)
    xs = np.concatenate([rng.normal(0, 100, 3000), rng.normal(0, 1e-5, 2000)]).astype(np.float32)
    for x in xs:
        assert O.f32_to_f16(float(x)) == int(np.float16(x).view(np.uint16))


# ------------------------------------------------------------------------------------------------ dequantisation goldens
@pytest.mark.parametrize("name", list(TYPES))
def test_dequant_matches_gguf_py_golden(name):
    v = golden()[name]
    raw = np.frombuffer(base64.b64decode(v["raw"]), np.uint8)
    want = np.frombuffer(base64.b64decode(v["expected"]), np.float32).reshape(v["rows"], v["cols"])
    got = O.dequant(TYPES[name], raw, v["rows"], v["cols"])
    # gguf-py computes in float32, the reference (and the oracle) in float64 then rounds: 1 ulp-ish, as
    # test/quant-vectors.test.js:21-23 allows
    ok = (got == want) | (np.abs(got - want) <= 2e-6 * np.abs(want) + 1e-30) | (np.isnan(got) & np.isnan(want))
    assert ok.all(), np.argwhere(~ok)[:5]


def test_unpack_scale_min_k4_hand_table():
    """test/quant-vectors.test.js:30-40: a hand-packed table round-trips (checked through Q4_K dequant of a block
    whose nibbles are all 1 and whose d = dmin = 1: value = sc - mn)."""
    sc = [1, 63, 32, 17, 0, 45, 63, 9]
    mn = [63, 0, 5, 40, 33, 2, 61, 50]
    q = np.zeros(12, np.uint8)
    for j in range(4):
        q[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        q[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        q[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[4:16] = q
    blk[16:] = 0x11
    out = O.dequant(G.Q4_K, blk, 1, 256)[0]
    for s in range(8):
        assert (out[s * 32:(s + 1) * 32] == sc[s] - mn[s]).all()


# ------------------------------------------------------------------------------------------------ Q8_0 / Q4_0 (test/quant.test.js:7-29)
def test_q8_0_layout_known_answer():
    x = (np.arange(32) - 16).astype(np.float32)
    q = O.quantize_q8_0(x)
    assert len(q) == 34
    d = float(np.frombuffer(q[:2].tobytes(), np.float16)[0])
    assert abs(d - 16 / 127) < 1e-4
    assert q[2:].view(np.int8)[0] == -127
    assert q[2:].view(np.int8)[16] == 0


def test_q8_0_round_trip_bound_and_zero_block():
    rng = np.random.default_rng(7)
    x = rng.normal(size=32 * 50).astype(np.float32)
    y = O.dequant(G.Q8_0, O.quantize_q8_0(x), 1, x.size)[0]
    for b in range(50):
        blk = x[b * 32:(b + 1) * 32]
        step = np.abs(blk).max() / 127
        assert (np.abs(blk - y[b * 32:(b + 1) * 32]) <= step * 0.51 + 1e-3 * np.abs(blk).max()).all()
    z = O.dequant(G.Q8_0, O.quantize_q8_0(np.zeros(32, np.float32)), 1, 32)[0]
    assert (z == 0).all()


def test_q4_0_round_trip_bound():
    rng = np.random.default_rng(8)
    x = rng.normal(size=32 * 40).astype(np.float32)
    y = O.dequant(G.Q4_0, O.quantize_q4_0(x), 1, x.size)[0]
    for b in range(40):
        blk = x[b * 32:(b + 1) * 32]
        step = np.abs(blk).max() / 8
        err = np.abs(blk - y[b * 32:(b + 1) * 32])
        # the largest-magnitude value maps to code 0 (exact up to the f16 rounding of d); its negation would need
        # code 16 and is clamped to 15
        assert err[np.argmax(np.abs(blk))] <= 1e-3 * np.abs(blk).max()
        assert (err <= step * 1.01 + 1e-6).all()
        assert (err[np.abs(blk) < 0.8 * np.abs(blk).max()] <= step * 0.51 + 1e-6).all()


# ------------------------------------------------------------------------------------------------ mulberry32
def test_mulberry32_matches_integer_recurrence():
    """mulberry32 written out with Python's unbounded integers and explicit 32-bit masks (Math.imul semantics)."""
    def ref(seed, n):
        a = seed & 0xFFFFFFFF
        out = []
        for _ in range(n):
            a = (a + 0x6D2B79F5) & 0xFFFFFFFF
            t = a
            t = ((t ^ (t >> 15)) * (t | 1)) & 0xFFFFFFFF
            t ^= (t + (((t ^ (t >> 7)) * (t | 61)) & 0xFFFFFFFF)) & 0xFFFFFFFF
            out.append(((t ^ (t >> 14)) & 0xFFFFFFFF) / 4294967296)
        return out

    for seed in (0, 1, 42, 0xFFFFFFFF, 123456789):
        r = O.Rng(seed)
        assert [r() for _ in range(50)] == ref(seed, 50)
    r = O.Rng(3)
    u = np.array([r() for _ in range(20000)])
    assert 0 <= u.min() and u.max() < 1 and abs(u.mean() - 0.5) < 0.01


# ------------------------------------------------------------------------------------------------ quantizeAct
def test_quantize_act_closed_form():
    rng = np.random.default_rng(11)
    x = rng.normal(0, 3, 32 * 64).astype(np.float32)
    x[5 * 32:6 * 32] = 0  # all-zero block
    q, d, s = O.quantize_act(x)
    for b in range(64):
        blk = x[b * 32:(b + 1) * 32].astype(np.float64)
        amax = np.abs(blk).max()
        assert d[b] == np.float32(amax / 127)
        qb = q[b * 32:(b + 1) * 32].astype(np.int64)
        assert s[b] == qb.sum()
        if amax == 0:
            assert (qb == 0).all()
            continue
        assert np.abs(qb).max() == 127 and qb[np.argmax(np.abs(blk))] == np.sign(blk[np.argmax(np.abs(blk))]) * 127
        assert (np.abs(qb * (amax / 127) - blk) <= amax / 127 / 2 * (1 + 1e-12)).all()


def test_quantize_act_rounds_half_away_from_zero():
    # amax = 127 -> scale 1, inv 1: x*inv lands exactly on k + 0.5
    x = np.zeros(32, np.float32)
    x[0] = 127
    x[1:7] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5]
    q, d, _ = O.quantize_act(x)
    assert list(q[1:7]) == [1, -1, 2, -2, 3, -3]


# ------------------------------------------------------------------------------------------------ matvec = brute force
def _rand_blocks(type_, rows, cols, seed):
    """Random raw blocks with moderate f16 scales (tools/random-blocks.js style, own code)."""
    rng = np.random.default_rng(seed)
    rb = G.row_size(type_, cols)
    raw = rng.integers(0, 256, size=rows * rb, dtype=np.uint8)
    _, bs, ts = G.TYPE_INFO[type_]
    blk = raw.reshape(-1, ts)
    f16 = lambda v: np.frombuffer(np.float16(v).tobytes(), np.uint8)
    for i in range(blk.shape[0]):
        d = 0.01 * (0.5 + rng.random())
        if type_ == G.Q6_K:
            blk[i, 208:210] = f16(d / 50)
        else:
            blk[i, 0:2] = f16(d)
            if type_ in (G.Q4_K, G.Q5_K):
                blk[i, 2:4] = f16(d * 2)
    return raw


@pytest.mark.parametrize("type_", [G.Q8_0, G.Q4_0, G.Q5_0, G.Q4_K, G.Q5_K, G.Q6_K, G.F32])
def test_matvec_equals_dequantize_then_dot(type_):
    rows, cols = 40, 512
    if type_ == G.F32:
        raw = np.random.default_rng(2).normal(0, 0.02, rows * cols).astype(np.float32).view(np.uint8)
    else:
        raw = _rand_blocks(type_, rows, cols, 3)
    x = np.random.default_rng(4).normal(size=cols).astype(np.float32)
    y = O.matvec(type_, raw, rows, cols, x)
    W = O.dequant(type_, raw, rows, cols).astype(np.float64)
    if type_ == G.F32:
        xa = x.astype(np.float64)
    else:
        q, d, _ = O.quantize_act(x)
        xa = q.astype(np.float64) * np.repeat(d.astype(np.float64), 32)
    want = W @ xa
    scale = np.abs(W).max() * np.abs(xa).sum()
    assert np.abs(y - want).max() <= 1e-6 * scale + 1e-30
    # a wrong block scale / index would be off by far more than f32 rounding
    assert np.abs(y - want).max() <= 4 * np.abs(want).max() * 2 ** -23 + 1e-12


def test_matvec_thread_count_invariant():
    raw = _rand_blocks(G.Q4_K, 300, 1024, 9)
    x = np.random.default_rng(1).normal(size=1024).astype(np.float32)
    O.set_threads(1)
    a = O.matvec(G.Q4_K, raw, 300, 1024, x)
    O.set_threads(4)
    b = O.matvec(G.Q4_K, raw, 300, 1024, x)
    O.set_threads(1)
    assert (a == b).all()


# ------------------------------------------------------------------------------------------------ sampler known answers
def test_distribution_known_answers():
    """test/spec-sampler.test.js:110-141."""
    l = np.array([2, 5, 1, 4, 3, 0, 4.5, -1], np.float32)
    d = O.Sampler(temperature=1, top_k=0, top_p=1).distribution(l)
    assert list(d.ids) == [1, 6, 3, 4, 0, 2, 5, 7]
    assert abs(d.probs.sum() - d.total) < 1e-12
    z = sum(math.exp(v - 5) for v in l)
    assert abs(O.prob_of(d, 3) - math.exp(4 - 5) / z) < 1e-12
    assert O.prob_of(d, 99) == 0
    d = O.Sampler(temperature=1, top_k=3, top_p=1).distribution(l)
    assert list(d.ids) == [1, 6, 3]
    assert abs(O.prob_of(d, 1) - 1 / (1 + math.exp(-0.5) + math.exp(-1))) < 1e-12
    d = O.Sampler(temperature=1, top_k=0, top_p=1, min_p=0.5).distribution(l)
    assert list(d.ids) == [1, 6]
    d = O.Sampler(temperature=1, top_k=0, top_p=0.5).distribution(l)
    assert list(d.ids) == [1, 6]
    d = O.Sampler(temperature=0).distribution(l)
    assert (list(d.ids), list(d.probs), d.total, d.greedy) == ([1], [1.0], 1.0, True)
    d = O.Sampler(temperature=0, repeat_penalty=2).distribution(l, [1])
    assert d.ids[0] == 6
    d = O.Sampler(temperature=1, top_k=0, top_p=1, presence_penalty=10).distribution(l, [1, 1, 6])
    assert list(d.ids[:2]) == [3, 4]


def test_draw_residual_known_answers():
    """test/spec-generate.test.js:243-261."""
    s = O.Sampler(temperature=1, top_k=0, top_p=1, seed=3)
    mk = lambda arr: s.distribution(np.log(np.array(arr, np.float32)))
    p, q = mk([0.5, 0.3, 0.15, 0.05]), mk([0.1, 0.6, 0.2, 0.1])
    for _ in range(200):
        assert O.draw_residual(s, p, q, 4) == 0
    p2, q2 = mk([0.4, 0.4, 0.1, 0.1]), mk([0.1, 0.2, 0.4, 0.3])
    c = [0, 0, 0, 0]
    N = 20000
    for _ in range(N):
        c[O.draw_residual(s, p2, q2, 4)] += 1
    assert c[2] + c[3] == 0
    assert abs(c[0] / N - 0.6) < 0.015
    same = {O.draw_residual(s, p, p, 4) for _ in range(300)}
    assert len(same) >= 3


def test_topk_heap_equals_sort_without_boundary_ties():
    rng = np.random.default_rng(0)
    for k in (1, 5, 40):
        l = rng.normal(size=5000).astype(np.float32)
        l[:50] = l[100]  # ties above the boundary are all kept
        ids, vals = O.topk_select(l, k)
        order = sorted(range(len(l)), key=lambda i: (-float(l[i]), i))[:k]
        if float(l[order[-1]]) != float(l[sorted(range(len(l)), key=lambda i: (-float(l[i]), i))[k]]):
            assert list(ids) == order


def test_draw_consumes_one_uniform_and_respects_total():
    s = O.Sampler(temperature=0.7, top_k=40, top_p=0.9, seed=9)
    l = np.random.default_rng(2).normal(size=1000).astype(np.float32)
    d = s.distribution(l)
    r = O.Rng(9)
    for _ in range(100):
        u = r() * d.total
        want = d.ids[-1]
        for i in range(len(d.ids)):
            u -= d.probs[i]
            if u <= 0:
                want = d.ids[i]
                break
        assert s.draw(d) == want


# ------------------------------------------------------------------------------------------------ forward = naive f64 forward
def _naive_logits(g, tokens):
    """Whole-sequence f64 forward over dequantised weights with unquantised activations (test/naive-forward.js:45-99)."""
    a = g.get("general.architecture")
    E = g.get(f"{a}.embedding_length")
    H = g.get(f"{a}.attention.head_count")
    HK = g.get(f"{a}.attention.head_count_kv")
    hd = g.get(f"{a}.attention.key_length")
    eps = g.get(f"{a}.attention.layer_norm_rms_epsilon")
    base = g.get(f"{a}.rope.freq_base")
    nl = g.get(f"{a}.block_count")

    def W(n):
        t = g.tensor(n)
        return O.dequant(t.type, np.asarray(g.data(n)), t.dims[1], t.dims[0]).astype(np.float64)

    def vec(n):
        return g.floats(n).astype(np.float64)

    def rms(x, w):
        return x / np.sqrt((x * x).mean() + eps) * w

    def rope(v, pos):
        half = hd // 2
        f = base ** (-2 * np.arange(half) / hd)
        c, s = np.cos(pos * f), np.sin(pos * f)
        a0, a1 = v[:half].copy(), v[half:].copy()
        return np.concatenate([a0 * c - a1 * s, a0 * s + a1 * c])

    emb = W("token_embd.weight")
    xs = [emb[t].copy() for t in tokens]
    for l in range(nl):
        p = f"blk.{l}."
        Wq, Wk, Wv, Wo = W(p + "attn_q.weight"), W(p + "attn_k.weight"), W(p + "attn_v.weight"), W(p + "attn_output.weight")
        qn, kn = vec(p + "attn_q_norm.weight"), vec(p + "attn_k_norm.weight")
        qs, ks, vs = [], [], []
        for pos, x in enumerate(xs):
            h = rms(x, vec(p + "attn_norm.weight"))
            q, k, v = Wq @ h, Wk @ h, Wv @ h
            qs.append([rope(rms(q[i * hd:(i + 1) * hd], qn), pos) for i in range(H)])
            ks.append([rope(rms(k[i * hd:(i + 1) * hd], kn), pos) for i in range(HK)])
            vs.append([v[i * hd:(i + 1) * hd] for i in range(HK)])
        out = []
        for pos, x in enumerate(xs):
            cat = []
            for h_ in range(H):
                kvh = h_ * HK // H
                sc = np.array([qs[pos][h_] @ ks[t][kvh] for t in range(pos + 1)]) / math.sqrt(hd)
                e = np.exp(sc - sc.max())
                pr = e / e.sum()
                cat.append(sum(pr[t] * vs[t][kvh] for t in range(pos + 1)))
            y = x + Wo @ np.concatenate(cat)
            h2 = rms(y, vec(p + "ffn_norm.weight"))
            gt, u = W(p + "ffn_gate.weight") @ h2, W(p + "ffn_up.weight") @ h2
            y = y + W(p + "ffn_down.weight") @ (gt / (1 + np.exp(-gt)) * u)
            out.append(y)
        xs = out
    outW = W("output.weight") if g.tensor("output.weight") else emb
    return [outW @ rms(x, vec("output_norm.weight")) for x in xs]


def test_forward_equals_naive_f64_on_f32_weights(tmp_path):
    """An F32-weight model (no activation quantisation in the reference path): oracle logits = naive f64 logits to
    f32 rounding (test/forward.test.js:99-118 allows 2e-4 of the max)."""
    from zerollm_amd import synth

    spec = synth.build_spec("qwen3", 64, 2, 4, 2, 32, 128, 300, 256, synth.all_type(G.F32), seed=5, std=0.05)
    path = str(tmp_path / "f32.gguf")
    synth.write_gguf(path, spec)
    g = G.read_gguf(path)
    toks = [3, 17, 250, 9, 9, 44, 120]
    m = O.OracleModel(g, ctx=64)
    got = [m.forward(t) for t in toks]
    want = _naive_logits(g, toks)
    for a, b in zip(got, want):
        assert np.abs(a - b).max() <= 1e-5 * np.abs(b).max()


def test_forward_q8_0_close_to_naive_and_f16_kv_close_to_f32(tiny_files):
    g = G.read_gguf(tiny_files[0])
    toks = [5, 900, 31000, 12, 77]
    m = O.OracleModel(g, ctx=64)
    got = [m.forward(t) for t in toks]
    want = _naive_logits(g, toks)
    for a, b in zip(got, want):
        cos = float(a @ b / np.linalg.norm(a) / np.linalg.norm(b))
        assert cos > 0.999
    m16 = O.OracleModel(g, ctx=64, kv="f16")
    got16 = [m16.forward(t) for t in toks]
    for a, b in zip(got, got16):
        assert float(a @ b / np.linalg.norm(a) / np.linalg.norm(b)) > 0.999


def test_oracle_truncate_replays_bit_exactly(tiny_files):
    m = O.OracleModel(tiny_files[0], ctx=64)
    toks = [1, 2, 3, 4, 5, 6]
    full = [m.forward(t) for t in toks]
    m.truncate(3)
    again = [m.forward(t) for t in toks[3:]]
    for a, b in zip(full[3:], again):
        assert (a == b).all()
