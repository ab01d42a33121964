"""The CPU baseline (oracle/pool_simd.c, oracle/pool.py): the AVX-512 VNNI restatement of the reference's worker-pool
pass must compute the oracle's arithmetic bit for bit, so its throughput is that of the same computation.
- tile kernels (Q8_0, Q4_K, Q6_K) and the scalar-row formats against the oracle's matvec, ragged row counts and batches;
- the model's batched passes (forwardBatch, src/compute/pool.js:145-160) against OracleModel's single-token forward,
  at ragged batch sizes and after truncation;
- speculative decoding over pool models (batched verify, src/model/speculative.js:39-48) against the single-token oracle
  models: the same tokens and the same per-cycle log, greedy and sampled."""
import numpy as np
import pytest

from oracle import oracle as O
from oracle import pool as P
from oracle.spec import plain, speculative
from zerollm_amd import gguf as G, synth

pytestmark = pytest.mark.skipif(not P.supported(), reason="CPU without AVX-512 VNNI")


def _raw(type_, rows, cols, seed):
    rng = np.random.default_rng(seed)
    if type_ == G.F32:
        return rng.normal(0, 0.05, (rows, cols)).astype(np.float32).view(np.uint8).ravel()
    raw = rng.integers(0, 256, size=rows * G.row_size(type_, cols), dtype=np.uint8)
    _, _, ts = G.TYPE_INFO[type_]
    blk = raw.reshape(-1, ts)
    f16 = lambda v: np.frombuffer(np.float16(v).tobytes(), np.uint8)
    for i in range(blk.shape[0]):  # finite scales
        d = 0.01 * (0.5 + rng.random())
        if type_ == G.Q6_K:
            blk[i, 208:210] = f16(d / 50)
        else:
            blk[i, 0:2] = f16(d)
            if type_ in (G.Q4_K, G.Q5_K):
                blk[i, 2:4] = f16(d * 2)
    return raw


@pytest.mark.parametrize("type_", [G.Q8_0, G.Q4_K, G.Q6_K, G.Q5_K, G.F32])
@pytest.mark.parametrize("rows,cols", [(37, 512), (300, 1024), (64, 4096)])
def test_tiles_equal_oracle_matvec(type_, rows, cols):
    raw = _raw(type_, rows, cols, rows + cols + type_)
    X = np.random.default_rng(rows).normal(0, 1, (7, cols)).astype(np.float32)
    X[1] *= 40.0
    X[2, :64] = 0
    want = np.stack([O.matvec(type_, raw, rows, cols, X[i]) for i in range(7)])
    for B, threads in ((1, 1), (5, 3), (7, 4)):
        got = P.matmul(type_, raw, rows, cols, X[:B], threads=threads)
        assert (got.view(np.uint32) == want[:B].view(np.uint32)).all(), (B, threads)


def _arrays(spec):
    return {t.name: synth.tensor_bytes(t, use_device=False) for t in spec.tensors}


@pytest.fixture(scope="module")
def models():
    q8, _ = synth.tiny_pair()
    q4km = synth.build_spec("qwen3", 512, 3, 8, 4, 64, 1536, 32000, 2048, synth.Q4_K_M, 7, name="tiny-q4km")
    return {"q8_0": (q8, _arrays(q8)), "q4_k_m": (q4km, _arrays(q4km))}


@pytest.mark.parametrize("which", ["q8_0", "q4_k_m"])
def test_batched_passes_equal_oracle_forward(models, which):
    spec, arr = models[which]
    src = O.ArraySource(spec, arr)
    ref = O.OracleModel(src, ctx=96, kv="f16", threads=2)
    pm = P.SimdPoolModel(src, ctx=96, threads=5)
    ids = synth.seeded_ids(40, 3, spec.vocab)
    want = np.stack([ref.forward(t) for t in ids])
    got, i = [], 0
    for n in (1, 3, 16, 5, 2, 13):
        got.append(pm.forward_batch(ids[i:i + n], logits="all"))
        i += n
    got = np.concatenate(got)
    assert (got.view(np.uint32) == want.view(np.uint32)).all()
    # the last-row mode, truncation and the single-token call
    pm.truncate(20)
    assert pm.pos == 20 and pm.tokens == ids[:20]
    last = pm.forward_batch(ids[20:25], logits="last")
    assert (last.view(np.uint32) == want[24].view(np.uint32)).all()
    pm.truncate(30)
    assert pm.forward_batch(ids[25:30], logits="none") is None
    assert (pm.forward(ids[30]).view(np.uint32) == want[30].view(np.uint32)).all()
    pm.close()
    ref.close()


def test_errors(models):
    spec, arr = models["q8_0"]
    pm = P.SimdPoolModel(O.ArraySource(spec, arr), ctx=20, threads=2)
    with pytest.raises(RuntimeError, match="batch of 17 tokens"):
        pm.forward_batch([1] * 17)
    with pytest.raises(RuntimeError, match="out of range"):
        pm.forward_batch([1, spec.vocab])
    pm.forward_batch([1] * 16, logits="none")
    with pytest.raises(RuntimeError, match="context full"):
        pm.forward_batch([1] * 5)
    assert pm.pos == 16
    pm.close()


@pytest.mark.parametrize("sampled", [False, True])
def test_speculative_over_pool_models_equals_oracle_models(sampled):
    t_spec, d_spec = synth.tiny_pair(layer_std=0.004)
    arr_t, arr_d = _arrays(t_spec), _arrays(d_spec)
    prompt = synth.seeded_ids(24, 11, t_spec.vocab)
    runs = []
    for kind in ("pool", "oracle"):
        if kind == "pool":
            t = P.SimdPoolModel(O.ArraySource(t_spec, arr_t), ctx=128, threads=4)
            d = P.SimdPoolModel(O.ArraySource(d_spec, arr_d), ctx=128, threads=3)
        else:
            t = O.OracleModel(O.ArraySource(t_spec, arr_t), ctx=128, kv="f16")
            d = O.OracleModel(O.ArraySource(d_spec, arr_d), ctx=128, kv="f16")
        smp = O.Sampler(temperature=0.8, top_k=40, top_p=0.95, seed=77) if sampled else None
        log, st = [], {}
        out = list(speculative(t, d, prompt, k=4, max_tokens=24, sample=smp, cycle_log=log, stats=st))
        runs.append((out, log, smp.rng.state if sampled else None))
        if kind == "oracle" and not sampled:
            t.reset()
            assert out == list(plain(t, prompt, 24))
        t.close()
        d.close()
    assert runs[0] == runs[1]
    assert len(runs[0][0]) == 24
    accepted = sum(a for _, _, a, _ in runs[0][1])
    assert accepted > 0, "the close pair accepts drafts"
