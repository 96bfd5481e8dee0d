"""The decoder workload (configs c4 / c5) on the CPU: the numpy oracle
(oracle/decoder.py) pinned against an independent torch float32 decoder
built on F.scaled_dot_product_attention, causality, RoPE's
relative-position property and GQA == MHA with duplicated KV heads; then
the product code (torch_spyre.examples.decoder) checked against the oracle
on the CPU, prefill and teacher-forced decode.
"""

import dataclasses

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import decoder as OD
from torch_spyre.examples import decoder as D

TINY = D.DecoderConfig(hidden=64, n_heads=4, n_kv_heads=2, head_dim=16, intermediate=96,
                       vocab=50, n_layers=2)


def _params(cfg, dtype=torch.float32, seed=3):
    return D.init_params(cfg, "cpu", dtype=dtype, seed=seed, std=0.2)


def _np(params):
    return {"embed": params["embed"].float().numpy(),
            "layers": [{k: v.float().numpy() for k, v in w.items()} for w in params["layers"]],
            "final_norm": params["final_norm"].float().numpy(),
            "lm_head": params["lm_head"].float().numpy()}


def _tokens(B, S, vocab, seed=5):
    return torch.randint(0, vocab, (B, S), generator=torch.Generator().manual_seed(seed))


def _sdpa_block(tokens, p, cfg):
    """Independent float32 decoder: SDPA with is_causal and enable_gqa."""
    h = p["embed"][tokens]
    B, S = tokens.shape
    pos = torch.arange(S, dtype=torch.float32)
    inv = 1.0 / cfg.rope_theta ** (torch.arange(0, cfg.head_dim, 2).float() / cfg.head_dim)
    ang = pos[:, None] * inv[None]
    cos, sin = ang.cos(), ang.sin()

    def rope(x):  # [B, H, S, D], complex-free rotate-half
        x1, x2 = x[..., : cfg.head_dim // 2], x[..., cfg.head_dim // 2:]
        return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], -1)

    for w in p["layers"]:
        x = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + cfg.eps) * w["attn_norm"]
        q = (x @ w["wq"].T).view(B, S, cfg.n_heads, -1).transpose(1, 2)
        k = (x @ w["wk"].T).view(B, S, cfg.n_kv_heads, -1).transpose(1, 2)
        v = (x @ w["wv"].T).view(B, S, cfg.n_kv_heads, -1).transpose(1, 2)
        a = F.scaled_dot_product_attention(rope(q), rope(k), v, is_causal=True, enable_gqa=True)
        h = h + a.transpose(1, 2).reshape(B, S, -1) @ w["wo"].T
        x = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + cfg.eps) * w["mlp_norm"]
        h = h + (F.silu(x @ w["wg"].T) * (x @ w["wu"].T)) @ w["wd"].T
    return h


def test_oracle_matches_independent_sdpa_decoder():
    p = _params(TINY)
    tok = _tokens(2, 12, TINY.vocab)
    want = _sdpa_block(tok, p, TINY).numpy()
    got = OD.block(tok.numpy(), _np(p), TINY, act=None)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4)


def test_oracle_is_causal():
    p = _np(_params(TINY))
    tok = _tokens(1, 10, TINY.vocab).numpy()
    h = OD.block(tok, p, TINY, act=None)
    tok2 = tok.copy()
    tok2[0, 6:] = (tok2[0, 6:] + 7) % TINY.vocab
    h2 = OD.block(tok2, p, TINY, act=None)
    np.testing.assert_array_equal(h[:, :6], h2[:, :6])
    assert np.abs(h[:, 6:] - h2[:, 6:]).max() > 1e-3


def test_rope_relative_position():
    rng = np.random.default_rng(0)
    q = rng.standard_normal((1, 1, 1, 16)).astype(np.float32)
    k = rng.standard_normal((1, 1, 1, 16)).astype(np.float32)

    def dot(m, n):
        cq, sq = OD.rope_tables(16, [m])
        ck, sk = OD.rope_tables(16, [n])
        return float(np.sum(OD._rope(q, cq, sq, None) * OD._rope(k, ck, sk, None)))

    assert dot(5, 2) == pytest.approx(dot(13, 10), rel=1e-4, abs=1e-5)
    assert dot(0, 0) == pytest.approx(float(np.sum(q * k)), rel=1e-5)
    assert dot(5, 2) != pytest.approx(dot(5, 3), rel=1e-3)


def test_gqa_equals_mha_with_duplicated_heads():
    rng = np.random.default_rng(1)
    q = rng.standard_normal((2, 5, 4, 8)).astype(np.float32)
    k = rng.standard_normal((2, 5, 2, 8)).astype(np.float32)
    v = rng.standard_normal((2, 5, 2, 8)).astype(np.float32)
    pos = np.arange(5)
    a = OD.attention(q, k, v, pos, pos)
    b = OD.attention(q, np.repeat(k, 2, axis=2), np.repeat(v, 2, axis=2), pos, pos)
    np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-6)


def test_product_block_matches_oracle_on_cpu():
    p = _params(TINY)
    tok = _tokens(2, 12, TINY.vocab)
    cos, sin = D.rope_tables(TINY, 12, "cpu", torch.float32)
    mask = D.causal_mask(TINY, 12, "cpu", torch.float32)
    h = D.block_forward(tok, p, cos, sin, mask, TINY)
    np.testing.assert_allclose(h.numpy(), OD.block(tok.numpy(), _np(p), TINY, act=None),
                               rtol=1e-4, atol=1e-4)


def test_product_generate_teacher_forced_matches_oracle_on_cpu():
    p = _params(TINY)
    prompt = _tokens(2, 9, TINY.vocab)
    teacher = _tokens(2, 4, TINY.vocab, seed=7)
    toks, logits = D.generate(prompt, p, TINY, 4, "cpu", teacher=teacher)
    want = OD.generate_teacher_forced(prompt.numpy(), teacher.numpy(), _np(p), TINY, act=None)
    np.testing.assert_allclose(logits.float().numpy(), want, rtol=1e-4, atol=1e-4)
    assert torch.equal(toks, logits[:-1].argmax(-1).T)


def test_static_decode_step_matches_eager_decode_on_cpu():
    p = _params(TINY)
    prompt = _tokens(2, 9, TINY.vocab)
    teacher = _tokens(2, 4, TINY.vocab, seed=7)
    _, a = D.generate(prompt, p, TINY, 4, "cpu", teacher=teacher)
    _, b = D.generate(prompt, p, TINY, 4, "cpu", teacher=teacher, decode_fn=D.decode_step_static)
    torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)


def test_fp16_rounding_model_tracks_fp32():
    # the act=fp16 oracle (the device's rounding points) stays within the
    # 1e-2 gate of the fp32 one at c4-like magnitudes
    cfg = dataclasses.replace(TINY, hidden=128, head_dim=32, intermediate=256)
    p = _np(D.init_params(cfg, "cpu", dtype=torch.float16, seed=4))
    tok = _tokens(1, 16, cfg.vocab).numpy()
    a = OD.block(tok, p, cfg, act=np.float16)
    b = OD.block(tok, p, cfg, act=None)
    np.testing.assert_allclose(a, b, rtol=1e-2, atol=1e-2)


# A shape at which every fused branch of the oracle's compiled-program mode
# is taken: head dim 128 with the stacked query rows of a KV head a multiple
# of 128 (fused prefill attention), rows % 256 == 0 with intermediate % 128
# and hidden % 64 (SwiGLU GEMM), and at most 8 rows in decode (SwiGLU weight
# stream).
FUSED = D.DecoderConfig(hidden=256, n_heads=2, n_kv_heads=1, head_dim=128, intermediate=256,
                        vocab=64, n_layers=2)


def _f32(tp):
    return {"embed": tp["embed"].float(), "final_norm": tp["final_norm"].float(),
            "lm_head": tp["lm_head"].float(),
            "layers": [{k: v.float() for k, v in w.items()} for w in tp["layers"]]}


def _sdpa_logits(tokens, p, cfg):
    h = _sdpa_block(tokens, p, cfg)
    x = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + cfg.eps) * p["final_norm"]
    return x @ p["lm_head"].T


def test_fused_mode_is_exact_math_without_rounding():
    # fused=True only moves rounding points: with act=None it is the same
    # float32 function as fused=False (prefill and teacher-forced decode)
    p = _np(D.init_params(FUSED, "cpu", seed=8))
    tok = _tokens(4, 64, FUSED.vocab).numpy()
    np.testing.assert_allclose(OD.block(tok, p, FUSED, act=None, fused=True),
                               OD.block(tok, p, FUSED, act=None, fused=False),
                               rtol=1e-5, atol=1e-6)
    # decode steps (<= 8 rows): RMSNorm and the residual adds folded into
    # the projections
    teacher = _tokens(4, 2, FUSED.vocab, seed=3).numpy()
    np.testing.assert_allclose(
        OD.generate_teacher_forced(tok[:, :16], teacher, p, FUSED, act=None, fused=True),
        OD.generate_teacher_forced(tok[:, :16], teacher, p, FUSED, act=None, fused=False),
        rtol=1e-4, atol=1e-5)


def test_decode_folds_change_only_rounding_points():
    # the decode-step folds (norm into the projection, residual into its
    # sums) move rounding points: one decode layer in fp16 differs from the
    # eager rounding model, by at most a few fp16 ulps of the activations
    p = _np(D.init_params(FUSED, "cpu", seed=8))
    w = p["layers"][0]
    h = np.random.default_rng(5).standard_normal((4, 1, FUSED.hidden)).astype(np.float16)
    pre = OD.layer(np.random.default_rng(6).standard_normal((4, 8, FUSED.hidden))
                   .astype(np.float16), w, FUSED, np.arange(8))[1]
    got, _ = OD.layer(h, w, FUSED, np.array([8]), kv_prefix=pre, fused=True)
    want, _ = OD.layer(h, w, FUSED, np.array([8]), kv_prefix=pre, fused=False)
    exact, _ = OD.layer(h, w, FUSED, np.array([8]), act=None, kv_prefix=pre, fused=False)
    assert np.abs(got - want).max() > 0
    np.testing.assert_allclose(got, exact, rtol=1e-2, atol=1e-2)
    assert np.abs(got - exact).mean() <= np.abs(want - exact).mean() * 1.05


def test_fused_rounding_model_tracks_independent_fp32_decoder():
    # the compiled-program rounding model (fp16 at each fused kernel's
    # output) against the independent SDPA decoder in float32, prefill at a
    # shape that takes every fused branch, within the 1e-2 gate; and it
    # rounds at fewer points than the eager model, so its mean error is no
    # larger
    tp = D.init_params(FUSED, "cpu", seed=8)
    p = _np(tp)
    tok = _tokens(4, 64, FUSED.vocab)
    want = _sdpa_block(tok, _f32(tp), FUSED).numpy()
    fused = OD.block(tok.numpy(), p, FUSED, act=np.float16, fused=True)
    eager = OD.block(tok.numpy(), p, FUSED, act=np.float16, fused=False)
    np.testing.assert_allclose(fused, want, rtol=1e-2, atol=1e-2)
    assert np.abs(fused - want).mean() <= np.abs(eager - want).mean() * 1.05
    # and the two rounding models are different programs
    assert np.abs(fused - eager).max() > 0


def test_fused_decode_tracks_independent_fp32_decoder():
    # teacher-forced decode in the compiled-program rounding model (SwiGLU
    # weight-stream branch, KV prefix) against the SDPA decoder run over the
    # whole sequence: the logits of step t are the last-position logits of
    # prompt + teacher[:t]
    tp = D.init_params(FUSED, "cpu", seed=9)
    tf = _f32(tp)
    prompt = _tokens(2, 64, FUSED.vocab, seed=11)
    teacher = _tokens(2, 3, FUSED.vocab, seed=12)
    got = OD.generate_teacher_forced(prompt.numpy(), teacher.numpy(), _np(tp), FUSED,
                                     fused=True)
    for t in range(4):
        seq = torch.cat([prompt, teacher[:, :t]], 1)
        want = _sdpa_logits(seq, tf, FUSED)[:, -1].numpy()
        np.testing.assert_allclose(got[t], want, rtol=1e-2, atol=1e-2)


HD128 = D.DecoderConfig(hidden=256, n_heads=4, n_kv_heads=2, head_dim=128, intermediate=192,
                        vocab=50, n_layers=2)


def test_fused_decode_attention_op_matches_plain_step_on_cpu():
    # decode_step_static through torch.ops.spyre.decode_attention (its CPU
    # chain) against the plain-op eager decode, float32
    p = _params(HD128)
    prompt = _tokens(2, 9, HD128.vocab)
    teacher = _tokens(2, 4, HD128.vocab, seed=7)
    _, a = D.generate(prompt, p, HD128, 4, "cpu", teacher=teacher)
    _, b = D.generate(prompt, p, HD128, 4, "cpu", teacher=teacher,
                      decode_fn=D.decode_step_static)
    torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("v_dim_major", [False, True])
def test_oracle_decode_step_attention_pinned(v_dim_major):
    # oracle.decoder.decode_step_attention (float32, act=None) against the
    # op-by-op chain of torch.ops.spyre.decode_attention on the CPU; a
    # rotation with the wrong sign and an off-by-one key range both fail
    import math

    import torch_spyre._inductor.customops  # noqa: F401

    g = torch.Generator().manual_seed(21)
    B, H, Hkv, L, Dh, pos = 2, 8, 2, 70, 128, 64
    qkv = torch.randn(B, (H + 2 * Hkv) * Dh, generator=g)
    kc = torch.randn(B, Hkv, L, Dh, generator=g)
    vc = torch.randn(B, Hkv, L, Dh, generator=g)
    ang = torch.arange(L, dtype=torch.float32)[:, None] * \
        (1e4 ** (-torch.arange(0, Dh, 2, dtype=torch.float32) / Dh))[None, :]
    ang = torch.cat([ang, ang], -1)
    cs, sn = ang.cos(), ang.sin()
    scale = 1.0 / math.sqrt(Dh)
    kt, vt = kc.clone(), (vc.transpose(2, 3).contiguous() if v_dim_major else vc.clone())
    out = torch.ops.spyre.decode_attention(qkv, cs, sn, torch.tensor([pos]), kt, vt, H, Hkv,
                                           scale, v_dim_major)
    o_want, k_want, v_want = OD.decode_step_attention(qkv.numpy(), cs.numpy(), sn.numpy(), pos,
                                                      kc.numpy(), vc.numpy(), H, Hkv, scale,
                                                      act=None)
    np.testing.assert_allclose(out.numpy(), o_want, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(kt.numpy(), k_want, rtol=1e-6, atol=1e-6)
    vt_kmaj = vt.transpose(2, 3) if v_dim_major else vt
    assert np.array_equal(vt_kmaj.numpy(), v_want)
    # planted mistakes: sin with the wrong sign; the new key left out
    bad, _, _ = OD.decode_step_attention(qkv.numpy(), cs.numpy(), -sn.numpy(), pos, kc.numpy(),
                                         vc.numpy(), H, Hkv, scale, act=None)
    assert not np.allclose(bad, out.numpy(), rtol=1e-3, atol=1e-3)
    bad2, _, _ = OD.decode_step_attention(qkv.numpy(), cs.numpy(), sn.numpy(), pos - 1,
                                          kc.numpy(), vc.numpy(), H, Hkv, scale, act=None)
    assert not np.allclose(bad2, out.numpy(), rtol=1e-3, atol=1e-3)


def test_prefill_chains_each_layer_norm_into_the_layer_before():
    # prefill hands each layer its input already normalised and takes the
    # next layer's normalised input (the LM head's, after the last layer)
    # from the layer before: the same arithmetic as normalising at the
    # start of each layer, so the logits are bit-identical on the CPU
    cfg = dataclasses.replace(TINY, n_layers=3)
    p = _params(cfg, torch.float32)
    tok = torch.randint(0, cfg.vocab, (2, 10), generator=torch.Generator().manual_seed(5))
    cos, sin = D.rope_tables(cfg, 10, "cpu", torch.float32)
    mask = D.causal_mask(cfg, 10, "cpu", torch.float32)
    cache = D.new_cache(cfg, 2, 10, "cpu", torch.float32)
    got = D.prefill(tok, p, cos, sin, mask, cache, cfg)
    h = F.embedding(tok, p["embed"])
    for w in p["layers"]:
        h = D.layer_forward(h, w, cos, sin, mask, cfg)  # normalises its own input
    want = D.lm_logits(h[:, -1], p, cfg)
    assert torch.equal(got, want)
    # and the cache holds the same K / V as the layers computed them
    cache2 = D.new_cache(cfg, 2, 10, "cpu", torch.float32)
    h = F.embedding(tok, p["embed"])
    for i, w in enumerate(p["layers"]):
        h = D.layer_forward(h, w, cos, sin, mask, cfg, cache2[i])
    for (k1, v1), (k2, v2) in zip(cache, cache2):
        assert torch.equal(k1, k2) and torch.equal(v1, v2)
