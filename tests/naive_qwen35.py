"""Independent whole-sequence Qwen3.5 (qwen35) forward for the tests, a numpy restatement of zerollm's deliberately
naive test oracle (test/naive-qwen35.js:1-221), NOT of the engine's token-by-token recurrence:
  - every position recomputed from the token ids in float64, no caches and no state objects;
  - the Gated DeltaNet evaluated in its parallel single-chunk "WY" form (chunkGatedDeltaRule,
    test/naive-qwen35.js:111-135): decay mask, forward substitution for (I + A)^-1, zero initial state;
  - the causal conv as a zero-padded sliding dot product over the whole sequence.
Weights come dequantised from the model's own tensors. The synthetic models are generated directly in GGUF order, so
value head h reads key head h % n_group, the order llama.cpp's converter produces (test/naive-qwen35.js undoes that
reorder and uses HF's repeat_interleave, which is the same mapping).
"""
from __future__ import annotations

import numpy as np


def _silu(z):
    return z / (1.0 + np.exp(-z))


def _sigmoid(z):
    return 1.0 / (1.0 + np.exp(-z))


def _softplus(z):
    return np.log1p(np.exp(z))


def _rms(x, w, eps):
    return x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps) * w


def _l2(x, eps=1e-6):
    return x / np.sqrt((x * x).sum(axis=-1, keepdims=True) + eps)


def chunk_gated_delta_rule(q, k, v, g, beta):
    """test/naive-qwen35.js:111-135 for one head: q, k [T][dk]; v [T][dv]; g [T] log decay; beta [T]."""
    T = q.shape[0]
    gc = np.cumsum(g)
    decay = np.exp(gc[:, None] - gc[None, :])
    attn = np.where(np.tril(np.ones((T, T), bool), -1), -(beta[:, None] * (k @ k.T) * decay), 0.0)
    for i in range(1, T):
        row = attn[i].copy()
        for j in range(i):
            row[j] = attn[i, j] + attn[i, :] @ attn[:, j]
        attn[i] = row
    attn += np.eye(T)
    value = attn @ (beta[:, None] * v)
    a = (q @ k.T) * decay * np.tril(np.ones((T, T)))
    return a @ value


def _rope(x, pos, n_rot, base):
    out = x.copy()
    half = n_rot // 2
    for i in range(half):
        th = pos * base ** (-2.0 * i / n_rot)
        out[..., i] = x[..., i] * np.cos(th) - x[..., i + half] * np.sin(th)
        out[..., i + half] = x[..., i + half] * np.cos(th) + x[..., i] * np.sin(th)
    return out


def naive_qwen35_logits(spec, W, V, tokens):
    """Logits for every position. W(name) -> float64 [rows][cols] dequantised matrix; V(name) -> float64 vector."""
    eps = float(np.float32(spec.rms_eps))
    dk, nK, nV = spec.d_state, spec.n_group, spec.dt_rank
    dv = spec.d_inner // nV
    key_dim = nK * dk
    hd, K = spec.head_dim, spec.conv_k
    E = W("token_embd.weight")
    xs = E[np.asarray(tokens)].copy()
    T = len(tokens)
    for l in range(spec.n_layer):
        p = f"blk.{l}."
        hs = _rms(xs, V(p + "attn_norm.weight"), eps)
        if (l + 1) % spec.interval != 0:
            raw = hs @ W(p + "attn_qkv.weight").T
            zs = hs @ W(p + "attn_gate.weight").T
            bs = hs @ W(p + "ssm_beta.weight").T
            as_ = hs @ W(p + "ssm_alpha.weight").T
            conv_w = V(p + "ssm_conv1d.weight").reshape(-1, K)
            mixed = np.zeros_like(raw)
            for t in range(T):
                s = np.zeros(raw.shape[1])
                for i in range(K):
                    tt = t - (K - 1) + i
                    if tt >= 0:
                        s += conv_w[:, i] * raw[tt]
                mixed[t] = _silu(s)
            core = np.zeros((T, spec.d_inner))
            A = V(p + "ssm_a")
            dt = V(p + "ssm_dt.bias")
            nw = V(p + "ssm_norm.weight")
            for hv in range(nV):
                kh = hv % nK
                qh = _l2(mixed[:, kh * dk:(kh + 1) * dk]) / np.sqrt(dk)
                kk = _l2(mixed[:, key_dim + kh * dk:key_dim + (kh + 1) * dk])
                vv = mixed[:, 2 * key_dim + hv * dv:2 * key_dim + (hv + 1) * dv]
                beta = _sigmoid(bs[:, hv])
                g = A[hv] * _softplus(as_[:, hv] + dt[hv])
                o = chunk_gated_delta_rule(qh, kk, vv, g, beta)
                o = o / np.sqrt((o * o).mean(axis=1, keepdims=True) + eps) * nw * _silu(zs[:, hv * dv:(hv + 1) * dv])
                core[:, hv * dv:(hv + 1) * dv] = o
            mixed_out = core @ W(p + "ssm_out.weight").T
        else:
            nH, nKV = spec.n_head, spec.n_head_kv
            qf = (hs @ W(p + "attn_q.weight").T).reshape(T, nH, 2 * hd)
            q = _rms(qf[:, :, :hd], V(p + "attn_q_norm.weight"), eps)
            gate = qf[:, :, hd:]
            k = _rms((hs @ W(p + "attn_k.weight").T).reshape(T, nKV, hd), V(p + "attn_k_norm.weight"), eps)
            v = (hs @ W(p + "attn_v.weight").T).reshape(T, nKV, hd)
            for t in range(T):
                q[t] = _rope(q[t], t, spec.n_rot, float(np.float32(spec.rope_base)))
                k[t] = _rope(k[t], t, spec.n_rot, float(np.float32(spec.rope_base)))
            out = np.zeros((T, nH, hd))
            grp = nH // nKV
            for t in range(T):
                for h in range(nH):
                    sc = (k[:t + 1, h // grp] @ q[t, h]) / np.sqrt(hd)
                    e = np.exp(sc - sc.max())
                    out[t, h] = (e / e.sum()) @ v[:t + 1, h // grp]
            mixed_out = (out * _sigmoid(gate)).reshape(T, nH * hd) @ W(p + "attn_output.weight").T
        xs = xs + mixed_out
        h2 = _rms(xs, V(p + "post_attention_norm.weight"), eps)
        ff = _silu(h2 @ W(p + "ffn_gate.weight").T) * (h2 @ W(p + "ffn_up.weight").T)
        xs = xs + ff @ W(p + "ffn_down.weight").T
    return _rms(xs, V("output_norm.weight"), eps) @ E.T


def chunked_gated_delta_rule(q, k, v, gam, beta, chunk=64):
    """The chunkwise form of one head's gated delta rule with the state carried between chunks (what a chunked
    prefill would run; test/naive-qwen35.js:111-135 is its single-chunk, zero-state case). S is [dv][dk], o_t = S_t q_t.
    Inside a chunk with decay products b_r = gam_1 ... gam_r the writes d_r solve (I + A) D = B, A[r][s] = beta_r
    (b_r / b_s) k_r.k_s (s < r), B_r = beta_r (v_r - b_r S_0 k_r); then o_r = b_r S_0 q_r + sum_{s<=r} (b_r / b_s)
    (k_s.q_r) d_s and S_C = b_C S_0 + sum_s (b_C / b_s) d_s k_s^T. Returns (outputs [T][dv], final state), float64."""
    from scipy.linalg import solve_triangular

    q, k, v, gam, beta = (np.asarray(x, np.float64) for x in (q, k, v, gam, beta))
    T, dk = k.shape
    dv = v.shape[1]
    S = np.zeros((dv, dk))
    out = np.zeros((T, dv))
    for c0 in range(0, T, chunk):
        Q, K, V, g, bt = q[c0:c0 + chunk], k[c0:c0 + chunk], v[c0:c0 + chunk], gam[c0:c0 + chunk], beta[c0:c0 + chunk]
        n = len(g)
        b = np.cumprod(g)
        ratio = b[:, None] / b[None, :]
        A = np.tril(bt[:, None] * ratio * (K @ K.T), -1)
        B = bt[:, None] * (V - b[:, None] * (K @ S.T))
        D = solve_triangular(np.eye(n) + A, B, lower=True, unit_diagonal=True)
        out[c0:c0 + n] = b[:, None] * (Q @ S.T) + (np.tril(ratio) * (Q @ K.T)) @ D
        S = b[-1] * S + ((b[-1] / b)[:, None] * D).T @ K
    return out, S
