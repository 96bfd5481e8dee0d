"""numpy restatement of the decoder workload (configs c4 / c5).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

The workload is defined by the benchmark configs, not by a reference file:
RMSNorm (eps 1e-5) -> Q/K/V projections -> RoPE (theta 1e4, rotate-half) ->
causal grouped-query attention (32 query heads over 8 KV heads, query head
h reads KV head h // 4) -> output projection + residual -> RMSNorm ->
SwiGLU MLP + residual; embedding gather in front, final RMSNorm and LM head
behind.  Arithmetic is float32 with float32 accumulation; with act=np.float16
intermediate values are rounded to fp16 where the device program holds an
fp16 tensor.  `fused` selects which program: False = eager (every op's
output is an fp16 tensor: RoPE rounds x*cos, rot*sin and their sum; the
scores round after the bmm and again after the scale; SiLU rounds before
the gate product), True = compiled (Inductor keeps values in registers
inside each fused kernel: RoPE and SiLU*up round once, the scale is applied
to the fp16 bmm output without another rounding; where the compiled program
runs attention as one fused kernel - prefill, head dim 128, the stacked
query rows of a KV head a multiple of 128 - the scores are not rounded at
all, only the probabilities before the second product; in a decode step
(one new position, head dim 128, at most 8 query heads per KV head) RoPE,
the cache append and attention are one kernel whose scores and
probabilities stay float32 (only the output rounds); where it runs the
gate / up projection and silu(gate) * up as one kernel - rows % 256 == 0,
intermediate % 128 == 0, hidden % 64 == 0, or at most 8 rows with
64 <= hidden <= 8192 - gate and up are not rounded either).  At most 8 rows
(a decode step) the compiled program also folds each RMSNorm into the
projection that reads it (rows <= 8, hidden % 8 == 0, 64 <= hidden <= 8192:
x * w rounds to fp16, the float32 sums are scaled by the row's
1 / rms(x), so the normalized activations are never rounded) and each
residual add into the projection that feeds it (at most 8 rows: h + x W^T
rounds once, from the float32 sums).

Pinned by tests/test_decoder.py against torch's CPU float32 ops with
F.scaled_dot_product_attention (is_causal, enable_gqa) as an independent
attention, causality (outputs at t do not change when later tokens do),
RoPE's relative-position property and GQA == MHA with duplicated K/V heads.
"""

from __future__ import annotations

import numpy as np

from . import ops as O


def _r(x, act):
    """x rounded to the activation type `act` (np.float16, "bfloat16", or
    None for float32)."""
    x = np.asarray(x, dtype=np.float32)
    return x if act is None else O._round_to(x, act)


def _linear(x, w, act):
    return _r(np.matmul(x.astype(np.float32), np.asarray(w, np.float32).T), act)


def _rmsnorm(x, w, eps, act):
    x = np.asarray(x, np.float32)
    ms = np.mean(x.astype(np.float64) ** 2, axis=-1, keepdims=True)
    return _r(x / np.sqrt(ms + eps).astype(np.float32) * np.asarray(w, np.float32), act)


def _norm_linear(h, nw, w, eps, act):
    """RMSNorm folded into a projection (float32 result, not rounded): the
    sums of fp16(h * nw) against w's rows, scaled by rsqrt(mean(h^2) + eps)
    of each row of h."""
    return O.rmsnorm_linear(h, nw, w, eps, act)


def _decode_fusions(rows, hidden, fused):
    """(norm folded into the projections, residual folded into the
    projections) for a compiled program over `rows` token rows."""
    small = fused and rows <= 8
    return small and hidden % 8 == 0 and 64 <= hidden <= 8192, small


def rope_tables(head_dim, positions, theta=1e4):
    """cos / sin [len(positions), head_dim]: angle_i = pos * theta^(-2i/d)
    in float32 (both halves equal), as the device tables are built."""
    inv = (1.0 / (np.float32(theta) ** (np.arange(0, head_dim, 2, dtype=np.float32)
                                         / np.float32(head_dim)))).astype(np.float32)
    ang = np.asarray(positions, np.float32)[:, None] * inv[None, :]
    ang = np.concatenate([ang, ang], axis=-1)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def _rope(x, cos, sin, act, fused=False):
    """x [B, S, H, D]; the rotate-half rotation of oracle.ops.rope."""
    half = x.shape[-1] // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    c = _r(cos, act)[None, :, None, :]
    s = _r(sin, act)[None, :, None, :]
    if fused:
        return _r(x * c + rot * s, act)
    return _r(_r(x * c, act) + _r(rot * s, act), act)


def attention(q, k, v, q_pos, k_pos, act=None, fused=False, scores_fp32=False,
              probs_fp32=False):
    """q [B, Sq, Hq, D], k / v [B, Sk, Hkv, D]; causal on absolute
    positions (key position <= query position).  Returns [B, Sq, Hq*D].
    scores_fp32: the scores stay float32 (a fused attention kernel);
    probs_fp32: so do the probabilities (the fused decode-step kernel,
    which normalises the float32 output sums once at the end)."""
    B, Sq, Hq, D = q.shape
    Hkv = k.shape[2]
    g = Hq // Hkv
    out = np.empty((B, Sq, Hq, D), np.float32)
    allowed = np.asarray(k_pos)[None, :] <= np.asarray(q_pos)[:, None]
    for b in range(B):
        for h in range(Hq):
            kh = h // g
            s = q[b, :, h].astype(np.float32) @ k[b, :, kh].astype(np.float32).T
            if not scores_fp32:
                s = _r(s, act)
            s = s * np.float32(1.0 / np.sqrt(D))
            if not fused and not scores_fp32:
                s = _r(s, act)
            s = np.where(allowed, s, np.float32(-np.inf))
            p = O.softmax(s, axis=-1)
            if not probs_fp32:
                p = _r(p, act)
            out[b, :, h] = _r(p @ v[b, :, kh].astype(np.float32), act)
    return out.reshape(B, Sq, Hq * D)


def layer(h, w, cfg, positions, act=np.float16, kv_prefix=None, fused=False):
    """One decoder layer.  h [B, S, hidden] at absolute `positions`;
    kv_prefix = (k, v) [B, P, Hkv, D] of earlier positions (decode).
    Returns (h_out, (k, v) of all positions)."""
    B, S, _ = h.shape
    H, Hkv, D = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    fold_norm, fold_res = _decode_fusions(B * S, cfg.hidden, fused)
    if fold_norm:
        q, k, v = (_r(_norm_linear(h, w["attn_norm"], w[n], cfg.eps, act), act)
                   for n in ("wq", "wk", "wv"))
    else:
        x = _rmsnorm(h, w["attn_norm"], cfg.eps, act)
        q, k, v = (_linear(x, w[n], act) for n in ("wq", "wk", "wv"))
    q, k, v = q.reshape(B, S, H, D), k.reshape(B, S, Hkv, D), v.reshape(B, S, Hkv, D)
    cos, sin = rope_tables(D, positions, cfg.rope_theta)
    q, k = _rope(q, cos, sin, act, fused), _rope(k, cos, sin, act, fused)
    k_pos = np.asarray(positions)
    if kv_prefix is not None:
        k = np.concatenate([kv_prefix[0], k], axis=1)
        v = np.concatenate([kv_prefix[1], v], axis=1)
        k_pos = np.arange(k.shape[1])
    # the compiled program's prefill attention is one fused kernel when its
    # shapes fit (head dim 128, stacked query rows per KV head % 128 == 0)
    fused_attn = fused and kv_prefix is None and D == 128 and (S * (H // Hkv)) % 128 == 0
    # its decode step (one new position) runs RoPE, the cache append and
    # attention as one kernel (torch.ops.spyre.decode_attention)
    fused_step = fused and kv_prefix is not None and S == 1 and D == 128 and H // Hkv <= 8
    a = attention(q, k, v, np.asarray(positions), k_pos, act, fused,
                  scores_fp32=fused_attn or fused_step, probs_fp32=fused_step)
    res_act = None if fold_res else act
    h = _r(h + _linear(a, w["wo"], res_act), act)
    # the compiled program's fused SwiGLU kernels keep gate / up in fp32
    # (tiled GEMM for whole 256-row blocks, weight stream for <= 8 rows)
    fused_mlp = fused and (((B * S) % 256 == 0 and cfg.intermediate % 128 == 0 and
                            cfg.hidden % 64 == 0) or
                           (B * S <= 8 and cfg.hidden % 8 == 0 and 64 <= cfg.hidden <= 8192))
    lin_act = None if fused_mlp else act
    if fold_norm:
        gte = _norm_linear(h, w["mlp_norm"], w["wg"], cfg.eps, act)
        up = _norm_linear(h, w["mlp_norm"], w["wu"], cfg.eps, act)
    else:
        x = _rmsnorm(h, w["mlp_norm"], cfg.eps, act)
        gte = _linear(x, w["wg"], lin_act)
        up = _linear(x, w["wu"], lin_act)
    m = _r((O.silu(gte) if fused else _r(O.silu(gte), act)) * up, act)
    return _r(h + _linear(m, w["wd"], res_act), act), (k, v)


def embed(tokens, table, act=np.float16):
    return _r(np.asarray(table, np.float32)[np.asarray(tokens)], act)


def block(tokens, params, cfg, act=np.float16, fused=False):
    """c4: embedding + layers over tokens [B, S] -> hidden [B, S, hidden]."""
    h = embed(tokens, params["embed"], act)
    pos = np.arange(np.asarray(tokens).shape[1])
    for w in params["layers"]:
        h, _ = layer(h, w, cfg, pos, act, fused=fused)
    return h


def logits(h_last, params, cfg, act=np.float16, fused=False):
    """Final RMSNorm + LM head on h_last [B, hidden]; fused: the compiled
    decode step's program (the norm folded into the head for <= 8 rows)."""
    if _decode_fusions(np.asarray(h_last).shape[0], cfg.hidden, fused)[0]:
        return _r(_norm_linear(h_last, params["final_norm"], params["lm_head"], cfg.eps, act),
                  act)
    x = _rmsnorm(h_last, params["final_norm"], cfg.eps, act)
    return _linear(x, params["lm_head"], act)


def generate_teacher_forced(prompt, teacher, params, cfg, act=np.float16, fused=False):
    """Prefill `prompt` [B, S], then feed `teacher` [B, T] one token at a
    time.  Returns logits [T+1, B, vocab] (prefill's last position first;
    its LM head runs eagerly, the decode steps' heads in the step's
    program)."""
    prompt = np.asarray(prompt)
    B, S = prompt.shape
    h = embed(prompt, params["embed"], act)
    caches = []
    for w in params["layers"]:
        h, kv = layer(h, w, cfg, np.arange(S), act, fused=fused)
        caches.append(kv)
    out = [logits(h[:, -1], params, cfg, act)]
    for t in range(np.asarray(teacher).shape[1]):
        h = embed(np.asarray(teacher)[:, t:t + 1], params["embed"], act)
        for i, w in enumerate(params["layers"]):
            h, caches[i] = layer(h, w, cfg, np.array([S + t]), act, kv_prefix=caches[i],
                                 fused=fused)
        out.append(logits(h[:, -1], params, cfg, act, fused=fused))
    return np.stack(out, 0)


def decode_step_attention(qkv, cos, sin, pos, k_cache, v_cache, n_heads, n_kv_heads, scale,
                          act=np.float16):
    """One decode step of attention with its cache append, as the fused
    decode-step kernel computes it: qkv [B, (H + 2 Hkv) * D] (query heads,
    then keys, then values), tables cos / sin [L, D] (already in the element
    type), position pos, caches k [B, Hkv, L, D] and v [B, Hkv, L, D]
    (key-major here).  Rotated q and k round once to `act`; scores,
    probabilities and output sums are float32; the output rounds once.
    Returns (out [B, H * D], k_cache', v_cache') with the new key / value at
    pos and keys 0..pos attended.  Pinned by tests/test_decoder.py against
    torch.ops.spyre.decode_attention's op-by-op CPU chain and against
    layer()'s decode-step attention."""
    qkv = np.asarray(qkv, np.float32)
    B = qkv.shape[0]
    H, Hkv = n_heads, n_kv_heads
    D = np.asarray(k_cache).shape[-1]
    q = qkv[:, :H * D].reshape(B, 1, H, D)
    k = qkv[:, H * D:(H + Hkv) * D].reshape(B, 1, Hkv, D)
    v = qkv[:, (H + Hkv) * D:].reshape(B, 1, Hkv, D)
    c = np.asarray(cos, np.float32)[pos:pos + 1]
    s = np.asarray(sin, np.float32)[pos:pos + 1]
    q = _rope(q, c, s, act, fused=True)
    k = _rope(k, c, s, act, fused=True)
    kc = np.array(k_cache, np.float32)
    vc = np.array(v_cache, np.float32)
    kc[:, :, pos] = k[:, 0]
    vc[:, :, pos] = v[:, 0]
    G = H // Hkv
    out = np.empty((B, H, D), np.float32)
    for b in range(B):
        for j in range(H):
            kh = j // G
            sc = (q[b, 0, j] @ kc[b, kh, :pos + 1].T) * np.float32(scale)
            p = O.softmax(sc[None, :], axis=-1)[0]
            out[b, j] = _r(p @ vc[b, kh, :pos + 1], act)
    return out.reshape(B, H * D), kc, vc
