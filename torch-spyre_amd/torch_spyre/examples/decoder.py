"""A random-init decoder (the benchmark's c4 / c5 workload) written with
plain torch ops, so the same code runs on the CPU and, eagerly or under
torch.compile, on the spyre device.

Shape: hidden 4096, 32 query heads / 8 KV heads of 128, RoPE (theta 1e4,
rotate-half), causal attention as bmm -> masked softmax -> bmm, SwiGLU MLP
of 12800, RMSNorm (eps 1e-5), vocab 49155, untied LM head.

Grouped-query attention is computed without copying K/V per query head:
the 4 query heads that share a KV head are stacked along the rows of one
bmm operand ([B*8, 4*S, 128] x [B*8, 128, S]), so each attention bmm is
4x taller and reads each K/V tile once; the causal mask repeats every S
rows.  Decoding uses a KV cache of one contiguous K buffer
[B, 8, max_len, 128] and one V buffer stored transposed, [B, 8, 128, max_len],
per layer: both attention products of a decode step then read their cache
operand along its contiguous dimension (scores: K rows; output: V^T rows),
which is the small-M streaming GEMM's layout.  The buffers are separate
tensors, so a compiled decode step scatters the new token's K/V into them
in place instead of copying an aliased cache.
"""

from __future__ import annotations

import dataclasses
import math
from typing import Optional

import torch
import torch.nn.functional as F

import torch_spyre._inductor.customops  # noqa: F401  (torch.ops.spyre.decode_attention)


@dataclasses.dataclass(frozen=True)
class DecoderConfig:
    hidden: int = 4096
    n_heads: int = 32
    n_kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 12800
    vocab: int = 49155
    n_layers: int = 40
    rope_theta: float = 1e4
    eps: float = 1e-5

    @property
    def group(self) -> int:
        return self.n_heads // self.n_kv_heads


C4 = DecoderConfig(n_layers=1)
C5 = DecoderConfig(n_layers=40)

LAYER_WEIGHTS = ("attn_norm", "wq", "wk", "wv", "wo", "mlp_norm", "wg", "wu", "wd")


def layer_shapes(cfg: DecoderConfig) -> dict:
    h, kv = cfg.hidden, cfg.n_kv_heads * cfg.head_dim
    return {"attn_norm": (h,), "wq": (cfg.n_heads * cfg.head_dim, h), "wk": (kv, h),
            "wv": (kv, h), "wo": (h, cfg.n_heads * cfg.head_dim), "mlp_norm": (h,),
            "wg": (cfg.intermediate, h), "wu": (cfg.intermediate, h),
            "wd": (h, cfg.intermediate)}


def init_params(cfg: DecoderConfig, device, dtype=torch.float16, seed: int = 0xAFFE,
                std: float = 0.02, pool_elems: Optional[int] = None) -> dict:
    """Random-init weights ~ N(0, std) (norm weights = ones), drawn on the
    CPU from a seeded generator and copied to `device`.

    With `pool_elems`, one pool of that many N(0, std) values is drawn once
    and every weight is a window of it at a seeded offset -- the same
    marginal distribution at a fraction of the host time, for throughput
    runs of the 40-layer model (16.7 GB of weights)."""
    g = torch.Generator().manual_seed(seed)
    pool = None
    if pool_elems:
        pool = (torch.randn(pool_elems, generator=g) * std).to(dtype)

    def draw(shape):
        n = math.prod(shape)
        if pool is None:
            return (torch.randn(*shape, generator=g) * std).to(dtype)
        reps = -(-n // pool.numel())
        src = pool if reps == 1 else pool.repeat(reps)
        off = int(torch.randint(0, src.numel() - n + 1, (1,), generator=g))
        return src[off:off + n].view(shape)

    params = {"embed": draw((cfg.vocab, cfg.hidden)).to(device), "layers": []}
    shp = layer_shapes(cfg)
    nq, nkv, ni = shp["wq"][0], shp["wk"][0], cfg.intermediate
    for _ in range(cfg.n_layers):
        # Q/K/V and gate/up weights live in one buffer each (one GEMM per
        # group reads the shared input once); the per-projection weights are
        # row views of them.
        wqkv = draw((nq + 2 * nkv, cfg.hidden)).to(device)
        wgu = draw((2 * ni, cfg.hidden)).to(device)
        lw = {"attn_norm": torch.ones(shp["attn_norm"], dtype=dtype).to(device),
              "wqkv": wqkv, "wq": wqkv[:nq], "wk": wqkv[nq:nq + nkv], "wv": wqkv[nq + nkv:],
              "wo": draw(shp["wo"]).to(device),
              "mlp_norm": torch.ones(shp["mlp_norm"], dtype=dtype).to(device),
              "wgu": wgu, "wg": wgu[:ni], "wu": wgu[ni:],
              "wd": draw(shp["wd"]).to(device)}
        params["layers"].append(lw)
    params["final_norm"] = torch.ones(cfg.hidden, dtype=dtype).to(device)
    params["lm_head"] = draw((cfg.vocab, cfg.hidden)).to(device)
    return params


def rope_tables(cfg: DecoderConfig, max_pos: int, device, dtype=torch.float16):
    """cos / sin [max_pos, head_dim] (both halves equal), angles in fp32."""
    d = cfg.head_dim
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    ang = torch.arange(max_pos, dtype=torch.float32)[:, None] * inv[None, :]
    ang = torch.cat([ang, ang], dim=-1)
    return ang.cos().to(dtype).to(device), ang.sin().to(dtype).to(device)


def causal_mask(cfg: DecoderConfig, seq: int, device, dtype=torch.float16):
    """Additive mask [group*seq, seq]: 0 where key <= query, -inf above the
    diagonal, repeated for the query heads stacked along the rows."""
    m = torch.full((seq, seq), float("-inf"), dtype=torch.float32).triu(1)
    return m.repeat(cfg.group, 1).to(dtype).to(device)


def _rotate_half(x):
    half = x.shape[-1] // 2
    return torch.cat([-x[..., half:], x[..., :half]], dim=-1)


def apply_rope(x, cos, sin):
    """x [B, S, H, D]; cos/sin [S, D] broadcast over batch and heads."""
    return x * cos[:, None, :] + _rotate_half(x) * sin[:, None, :]


def _attention(q, k, v, cfg: DecoderConfig, mask):
    """q [B, Sq, 32, D], k / v [B, 8, Sk, D] -> [B*Sq, 32*D] (2-D, so the
    output projection is one GEMM with the weight read once)."""
    B, Sq = q.shape[0], q.shape[1]
    kv, g, D = cfg.n_kv_heads, cfg.group, cfg.head_dim
    qg = q.view(B, Sq, kv, g, D).permute(0, 2, 3, 1, 4).reshape(B * kv, g * Sq, D)
    kk = k.reshape(B * kv, -1, D)
    vv = v.reshape(B * kv, -1, D)
    s = torch.bmm(qg, kk.transpose(1, 2)) * (1.0 / math.sqrt(D))
    if mask is not None:
        s = s + mask
    p = torch.softmax(s, dim=-1)
    o = torch.bmm(p, vv)  # [B*kv, g*Sq, D]
    return o.view(B, kv, g, Sq, D).permute(0, 3, 1, 2, 4).reshape(B * Sq, kv * g * D)


def _qkv(x, w: dict, cfg: DecoderConfig):
    """Q, K, V projections of x [..., hidden]: one GEMM over the fused
    weight when the layer has one."""
    if "wqkv" in w:
        nq, nkv = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
        qkv = F.linear(x, w["wqkv"])
        return qkv[..., :nq], qkv[..., nq:nq + nkv], qkv[..., nq + nkv:]
    return F.linear(x, w["wq"]), F.linear(x, w["wk"]), F.linear(x, w["wv"])


def _mlp(x, w: dict, cfg: DecoderConfig):
    """SwiGLU: down(silu(gate(x)) * up(x)), gate and up as one GEMM when
    the layer has the fused weight."""
    if "wgu" in w:
        gu = F.linear(x, w["wgu"])
        g, u = gu[..., :cfg.intermediate], gu[..., cfg.intermediate:]
    else:
        g, u = F.linear(x, w["wg"]), F.linear(x, w["wu"])
    return F.linear(F.silu(g) * u, w["wd"])


def layer_forward(h, w: dict, cos, sin, mask, cfg: DecoderConfig, cache_kv=None, x=None,
                  next_norm=None):
    """One decoder layer on h [B, S, hidden] (prefill).  If `cache_kv` is
    given (the layer's (K, V) cache buffers [B, 8, max_len, D]), K/V of
    positions [0, S) are written into it.  `x`, if given, is h normalised
    with this layer's attention norm (computed by the layer before); with
    `next_norm` the layer returns (output, output normalised with that
    weight), so its last residual add and the next layer's first RMSNorm
    are one kernel of this layer's compiled graph."""
    B, S, _ = h.shape
    if x is None:
        x = F.rms_norm(h, (cfg.hidden,), w["attn_norm"], cfg.eps)
    q, k, v = _qkv(x, w, cfg)
    q = q.reshape(B, S, cfg.n_heads, cfg.head_dim)
    k = k.reshape(B, S, cfg.n_kv_heads, cfg.head_dim)
    v = v.reshape(B, S, cfg.n_kv_heads, cfg.head_dim)
    q = apply_rope(q, cos[:S], sin[:S])
    k = apply_rope(k, cos[:S], sin[:S]).transpose(1, 2)
    v = v.transpose(1, 2)
    if cache_kv is not None:
        cache_kv[0][:, :, :S].copy_(k)
        cache_kv[1][:, :, :, :S].copy_(v.transpose(2, 3))
    h = h + F.linear(_attention(q, k, v, cfg, mask), w["wo"]).view(B, S, cfg.hidden)
    x = F.rms_norm(h, (cfg.hidden,), w["mlp_norm"], cfg.eps)
    h = h + _mlp(x, w, cfg)
    if next_norm is None:
        return h
    return h, F.rms_norm(h, (cfg.hidden,), next_norm, cfg.eps)


def block_forward(tokens, params: dict, cos, sin, mask, cfg: DecoderConfig):
    """c4: embedding + the model's layers over tokens [B, S] -> hidden."""
    h = F.embedding(tokens, params["embed"])
    for w in params["layers"]:
        h = layer_forward(h, w, cos, sin, mask, cfg)
    return h


def new_cache(cfg: DecoderConfig, batch: int, max_len: int, device, dtype=torch.float16):
    """Per layer, a zeroed K buffer [batch, 8, max_len, head_dim] and a
    zeroed transposed V buffer [batch, 8, head_dim, max_len]."""
    kshape = (batch, cfg.n_kv_heads, max_len, cfg.head_dim)
    vshape = (batch, cfg.n_kv_heads, cfg.head_dim, max_len)
    return [(torch.zeros(kshape, dtype=dtype, device=device),
             torch.zeros(vshape, dtype=dtype, device=device)) for _ in range(cfg.n_layers)]


def lm_logits(h_last, params: dict, cfg: DecoderConfig):
    """Final RMSNorm + LM head on h_last [B, hidden] -> logits [B, vocab]."""
    x = F.rms_norm(h_last, (cfg.hidden,), params["final_norm"], cfg.eps)
    return F.linear(x, params["lm_head"])


def prefill(tokens, params: dict, cos, sin, mask, cache, cfg: DecoderConfig, layer_fn=None):
    """Runs the prompt tokens [B, S] through every layer, filling the KV
    cache, and returns the logits of the last position [B, vocab]."""
    layer_fn = layer_fn or layer_forward
    h = F.embedding(tokens, params["embed"])
    layers = params["layers"]
    # Each layer also normalises its output for the next one (the last for
    # the LM head), so every call has the same arguments: one compiled
    # graph serves all layers.
    x = F.rms_norm(h, (cfg.hidden,), layers[0]["attn_norm"], cfg.eps)
    for i, w in enumerate(layers):
        nxt = layers[i + 1]["attn_norm"] if i + 1 < len(layers) else params["final_norm"]
        h, x = layer_fn(h, w, cos, sin, mask, cfg, cache[i], x, nxt)
    return F.linear(x[:, -1], params["lm_head"])


def decode_step(tokens, pos: int, params: dict, cos, sin, cache, cfg: DecoderConfig):
    """One token per sequence (tokens [B]) at position `pos`: appends its
    K/V to the cache and returns the logits [B, vocab]."""
    B = tokens.shape[0]
    h = F.embedding(tokens, params["embed"]).view(B, 1, cfg.hidden)
    c, s = cos[pos:pos + 1], sin[pos:pos + 1]
    for i, w in enumerate(params["layers"]):
        x = F.rms_norm(h, (cfg.hidden,), w["attn_norm"], cfg.eps)
        q, k, v = _qkv(x, w, cfg)
        q = apply_rope(q.reshape(B, 1, cfg.n_heads, cfg.head_dim), c, s)
        k = apply_rope(k.reshape(B, 1, cfg.n_kv_heads, cfg.head_dim), c, s)
        v = v.reshape(B, 1, cfg.n_kv_heads, cfg.head_dim)
        kc, vc = cache[i]
        kc[:, :, pos:pos + 1].copy_(k.transpose(1, 2))
        vc[:, :, :, pos:pos + 1].copy_(v.permute(0, 2, 3, 1))
        kc, vc = kc[:, :, :pos + 1], vc[:, :, :, :pos + 1].transpose(2, 3)
        h = h + F.linear(_attention(q, kc, vc, cfg, None), w["wo"]).view(B, 1, cfg.hidden)
        x = F.rms_norm(h, (cfg.hidden,), w["mlp_norm"], cfg.eps)
        h = h + _mlp(x, w, cfg)
    return lm_logits(h[:, 0], params, cfg)


def decode_step_static(tokens, pos, params: dict, cos, sin, cache, cfg: DecoderConfig,
                       fused_attention: bool = True):
    """decode_step with every shape fixed, for torch.compile: `pos` is a
    one-element int64 tensor on the device, the new K/V are scattered into
    the cache at `pos` and attention runs over the cache with keys after
    `pos` masked out, so one compiled graph serves every step.

    With `fused_attention` (and a fused Q/K/V weight) RoPE, the cache
    append and attention of a layer are one call of the spyre op
    torch.ops.spyre.decode_attention (on spyre one kernel that reads only
    the keys up to `pos`; elsewhere the same op-by-op chain as below);
    otherwise they are written out as plain torch ops over the whole cache
    length."""
    B = tokens.shape[0]
    L = cache[0][0].shape[2]  # K buffer [B, 8, max_len, D]
    h = F.embedding(tokens, params["embed"]).view(B, 1, cfg.hidden)
    c, s = cos.index_select(0, pos), sin.index_select(0, pos)
    keys = torch.arange(L, device=tokens.device)
    mask = torch.where(keys <= pos, 0.0, float("-inf")).to(h.dtype)
    for i, w in enumerate(params["layers"]):
        x = F.rms_norm(h, (cfg.hidden,), w["attn_norm"], cfg.eps)
        if fused_attention and "wqkv" in w and cfg.head_dim == 128:
            kc, vc = cache[i]
            qkv = F.linear(x, w["wqkv"]).view(B, -1)
            a = torch.ops.spyre.decode_attention(qkv, cos, sin, pos, kc, vc, cfg.n_heads,
                                                 cfg.n_kv_heads, 1.0 / math.sqrt(cfg.head_dim),
                                                 True)
            h = h + F.linear(a, w["wo"]).view(B, 1, cfg.hidden)
            x = F.rms_norm(h, (cfg.hidden,), w["mlp_norm"], cfg.eps)
            h = h + _mlp(x, w, cfg)
            continue
        q, k, v = _qkv(x, w, cfg)
        q = apply_rope(q.reshape(B, 1, cfg.n_heads, cfg.head_dim), c, s)
        k = apply_rope(k.reshape(B, 1, cfg.n_kv_heads, cfg.head_dim), c, s)
        v = v.reshape(B, 1, cfg.n_kv_heads, cfg.head_dim)
        kc, vc = cache[i]
        kc.index_copy_(2, pos, k.transpose(1, 2))
        vc.index_copy_(3, pos, v.permute(0, 2, 3, 1))
        h = h + F.linear(_attention(q, kc, vc.transpose(2, 3), cfg, mask),
                         w["wo"]).view(B, 1, cfg.hidden)
        x = F.rms_norm(h, (cfg.hidden,), w["mlp_norm"], cfg.eps)
        h = h + _mlp(x, w, cfg)
    return lm_logits(h[:, 0], params, cfg)


def generate(prompt, params: dict, cfg: DecoderConfig, steps: int, device, layer_fn=None,
             teacher=None, decode_fn=None, use_graph=False):
    """Greedy decoding: prefill `prompt` [B, S], then `steps` decode steps.
    Returns (the argmax token of each step [B, steps], the logits that chose
    them [steps+1, B, vocab]).  With `teacher` ([B, steps] tokens) those
    tokens are fed back instead of the argmax (teacher forcing), so the
    logits of a device run and a CPU run can be compared step by step.
    `decode_fn` (e.g. torch.compile(decode_step_static)) replaces the
    eager decode step; its position tensor lives on the device and is
    advanced there, so no step waits on the host.  With `use_graph` the
    decode step (decode_fn, the argmax and the position update) is captured
    once into a HIP graph of the spyre stream and each step is one replay."""
    B, S = prompt.shape
    dt = params["embed"].dtype
    cos, sin = rope_tables(cfg, S + steps, device, dt)
    cache = new_cache(cfg, B, S + steps, device, dt)
    logits = [prefill(prompt, params, cos, sin, causal_mask(cfg, S, device, dt), cache, cfg,
                      layer_fn)]
    out = []
    pos = torch.full((1,), S, dtype=torch.int64).to(device) if decode_fn is not None else None
    if use_graph and steps > 0:
        if decode_fn is None:
            raise ValueError("use_graph needs a decode_fn with static shapes")
        return _generate_graph(logits, pos, params, cfg, steps, cos, sin, cache, decode_fn,
                               teacher)
    for t in range(steps):
        nxt = logits[-1].argmax(-1)
        out.append(nxt)
        feed = nxt if teacher is None else teacher[:, t]
        if decode_fn is None:
            logits.append(decode_step(feed, S + t, params, cos, sin, cache, cfg))
        else:
            logits.append(decode_fn(feed, pos, params, cos, sin, cache, cfg))
            pos.add_(1)
    return torch.stack(out, 1), torch.stack(logits, 0)


def _generate_graph(logits, pos, params, cfg, steps, cos, sin, cache, decode_fn, teacher):
    import torch_spyre.graphs as graphs

    feed = logits[0].argmax(-1)
    out = [feed.clone()]
    if teacher is not None:
        feed.copy_(teacher[:, 0])
    # one real step outside the capture loads every kernel; it writes the
    # cache at `pos` exactly as the first replay will
    decode_fn(feed, pos, params, cos, sin, cache, cfg)
    g = graphs.SpyreGraph()
    with graphs.graph(g):
        step_logits = decode_fn(feed, pos, params, cos, sin, cache, cfg)
        step_arg = step_logits.argmax(-1)
        pos.add_(1)
    for t in range(steps):
        g.replay()
        logits.append(step_logits.clone())
        if t + 1 < steps:
            out.append(step_arg.clone())
            feed.copy_(step_arg if teacher is None else teacher[:, t + 1])
    g.reset()
    return torch.stack(out, 1), torch.stack(logits, 0)
