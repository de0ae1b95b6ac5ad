"""numpy restatement of the denoising step around the blocks.

TEST INFRASTRUCTURE ONLY: imported by tests/, never by the product library.

Follows QwenImageTransformerQuantized (src/quantized_transformer.rs:311-551),
its prefix fill prefix_kv (:359-392) and zero_modulation (:334-343), the
FlowMatchEuler scheduler (src/scheduler.rs:24-126) and the CFG combine of the
sampling loop (src/pipeline.rs:168-197). The blocks run through the pinned C
oracle (oracle.block_forward); the global linears through oracle.qmatmul in
exact mode (f64 accumulation of exactly dequantized weights), as the reference
runs its F32-stored global weights; SiLU and GELU(tanh) in f64.

Pinning (tests/test_step_cpu.py, tests/test_gpu_step.py):
- flow_match_sigmas: the reference's own scheduler tests (src/scheduler.rs:148-185),
  the telescoping sum of the Euler steps (sum dt = -sigma_0), the closed form of
  the exponential shift written another way (t e^mu / (t e^mu + 1 - t)), and
  mu = 0.5 exactly at 256 image tokens;
- layout pieces: the reference's layout tests (src/joint_layout.rs:133-164) and
  the image ids of oracle.joint_layout;
- silu / gelu_tanh: the odd-part identities f(x) - f(-x) = x and f(0) = 0,
  and the tanh-form GELU(1);
- the timestep embedding (oracle.timestep_embedding): the closed form
  [cos(1000 t f_i) | sin(1000 t f_i)], f_i = 10000^(-i/128), at t up to 1, the
  known points t = 0.001 (angle 1 rad) and t = pi/2000 (angle pi/2), the
  angle ratio 10000^(-1/128) and the angles recovered by atan2; the t = 0
  constant [1 x 128, 0 x 128] the reference states
  (src/quantized_transformer.rs:337);
- time_embed, modulation, txt_in and final_layer with special weights whose
  outputs have closed forms: identity linears give silu(t); modulation rows
  [I; 2I; 0; -I] give the four chunks of silu(t_emb); the text embedder gives
  gelu_tanh(x / rms(x) * (1 + stored)); the final layer's rows have mean 0 and
  spread |1 + c| when norm_out maps silu(t_emb) to the constant c;
- the composition: with no blocks, identity img_in / proj_out and a zero
  norm_out the forward returns LayerNorm(latents), and a zero proj_out gives
  zero velocity.
"""
from __future__ import annotations

import numpy as np

import oracle as O

TIME_DIM = 256


def silu(x):
    x = np.asarray(x, dtype=np.float64)
    return x / (1.0 + np.exp(-x))


def gelu_tanh(x):
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def linear(w, x):
    """Bias-free Linear (src/quantized_transformer.rs:14-33): w = (type, bytes, rows=out, cols=in)."""
    t, data, rows, cols = w
    x = np.asarray(x, dtype=np.float32)
    lead = x.shape[:-1]
    return O.qmatmul(t, data, rows, cols, x.reshape(-1, cols), O.EXACT).reshape(*lead, rows)


def time_embed(g, t_sin):
    """QwenTimestepEmbedder::forward (:50-54): linear_2(silu(linear_1(t)))."""
    return linear(g["t_linear_2"], silu(linear(g["t_linear_1"], t_sin)))


def modulation(g, temb):
    """Modulation::forward (:226-228) -> [B, 1, 4 hidden]."""
    return linear(g["modulation"], silu(temb))[:, None, :]


def zero_sinusoid(batch):
    z = np.zeros((batch, TIME_DIM), np.float32)
    z[:, :TIME_DIM // 2] = 1.0
    return z


def txt_in(g, txt):
    """QTextEmbedder::forward (:76-81): RMSNorm(scale = stored + 1) -> in_layer -> GELU(tanh) -> out_layer."""
    wn = O.dequantize(g["txt_norm"][0], g["txt_norm"][1], g["txt_norm"][2] * g["txt_norm"][3]) + 1.0
    x = O.rmsnorm(np.asarray(txt, np.float32), wn.astype(np.float32))
    return linear(g["txt_out"], gelu_tanh(linear(g["txt_in"], x)))


def final_layer(g, h, temb):
    """FinalLayer::forward (:300-309) then proj_out (:545)."""
    scale = linear(g["norm_out"], silu(temb))  # [B, hidden]
    out = np.empty_like(np.asarray(h, np.float32))
    for b in range(h.shape[0]):
        out[b] = O.layernorm_mod(h[b], scale[b])
    return linear(g["proj_out"], out)


def model_forward(cfg, g, blocks, latents, t_sin, pe, kcache=None, vcache=None, key_valid=None, mode=O.CANDLE):
    """The cached step of forward_conditioned (:471-551): latents [B,S,C], t_sin [B,256], pe [S,128],
    kcache/vcache per layer bf16 [B,H,P,D] (or None), key_valid [B, P+S] or None. Returns pred [B,S,C]."""
    temb = time_embed(g, t_sin)
    mod = modulation(g, temb)
    h = linear(g["img_in"], latents)
    b, s, _ = h.shape
    mask = None
    if key_valid is not None:
        mask = np.repeat(np.asarray(key_valid, np.uint8)[:, None, :], s, axis=1)
    for i, w in enumerate(blocks):
        kp = None if kcache is None else kcache[i]
        vp = None if vcache is None else vcache[i]
        h, _, _ = O.block_forward(cfg, w, h, mod, pe, kp, vp, mask=mask, mode=mode)
    return final_layer(g, h, temb)


def model_forward_rows(cfg, g, blocks, latents, t_sin, pe, rows, kcache=None, vcache=None, mode=O.CANDLE):
    """model_forward for the flat token rows `rows` of [B*S] only: every block
    but the last over all tokens (the last block needs every token's K and V),
    the last one through oracle.block_forward_rows, then the final layer on
    those rows. Bit-identical to the same rows of model_forward. Returns
    pred [len(rows), C]."""
    temb = time_embed(g, t_sin)
    mod = modulation(g, temb)
    h = linear(g["img_in"], latents)
    b, s, _ = h.shape
    for i, w in enumerate(blocks[:-1]):
        kp = None if kcache is None else kcache[i]
        vp = None if vcache is None else vcache[i]
        h, _, _ = O.block_forward(cfg, w, h, mod, pe, kp, vp, mode=mode)
    rows = np.asarray(rows)
    if blocks:
        i = len(blocks) - 1
        kp = None if kcache is None else kcache[i]
        vp = None if vcache is None else vcache[i]
        hr, _, _ = O.block_forward_rows(cfg, blocks[-1], h, mod, pe, rows, kp, vp, mode=mode)
    else:
        hr = h.reshape(b * s, -1)[rows]
    out = np.empty((len(rows), h.shape[-1]), np.float32)
    scale = linear(g["norm_out"], silu(temb))
    for j, r in enumerate(rows):
        out[j] = O.layernorm_mod(hr[j][None], scale[r // s])[0]
    return linear(g["proj_out"], out)


def assemble(txt_h, cond_h, pieces):
    """JointLayout::assemble narrowed to the prefix (src/joint_layout.rs:112-126)."""
    parts = [(txt_h if kind == 0 else cond_h)[:, st:st + n] for kind, st, n in pieces]
    return np.concatenate(parts, axis=1)


def prefix_fill(cfg, g, blocks, txt, cond, pieces, image_ids, key_valid, pe, mode=O.CANDLE):
    """prefix_kv (:359-392): returns per layer (k, v) as bf16 [B,H,P,D] (to_cache_entry)."""
    txt_h = txt_in(g, txt) if "txt_in" in g else np.asarray(txt, np.float32)
    cond_h = linear(g["img_in"], cond) if cond is not None else None
    x = assemble(txt_h, cond_h, pieces)
    b, p, _ = x.shape
    mod = modulation(g, time_embed(g, zero_sinusoid(1)))
    mask = O.block_causal_mask(np.asarray(image_ids, np.int64))[None]
    if key_valid is not None:
        mask = mask * np.asarray(key_valid, np.uint8)[:, None, :]
    out = []
    for w in blocks:
        x, k, v = O.block_forward(cfg, w, x, np.repeat(mod, b, axis=0), pe, mask=mask, mode=mode)
        out.append((O.f32_to_bf16(k), O.f32_to_bf16(v)))
    return out


def flow_match_sigmas(steps, image_seq_len):
    """FlowMatchEuler::new (src/scheduler.rs:24-37), float32 in the reference's order."""
    f = np.float32
    base_shift, max_shift, shift_terminal = f(0.5), f(0.9), f(0.02)
    m = (max_shift - base_shift) / (f(8192) - f(256))
    bb = base_shift - m * f(256)
    mu = f(image_seq_len) * m + bb
    start, end = f(1.0), f(1.0) / f(steps)
    e_mu = np.exp(mu, dtype=np.float32)
    sig = []
    for i in range(steps):
        t = start if steps <= 1 else start + (end - start) * f(i) / f(steps - 1)
        sig.append(e_mu / (e_mu + (f(1.0) / t - f(1.0))))
    sig = np.array(sig, dtype=np.float32)
    scale = (f(1.0) - sig[-1]) / (f(1.0) - shift_terminal)
    return (f(1.0) - (f(1.0) - sig) / scale).astype(np.float32)


def euler_dt(sigmas, i):
    """FlowMatchEuler::step's dt (src/scheduler.rs:55-59)."""
    return float(sigmas[i + 1] - sigmas[i]) if i + 1 < len(sigmas) else -float(sigmas[i])


def cfg_combine(cond, neg, scale):
    """neg + scale * (cond - neg) (src/pipeline.rs:182-184)."""
    return neg + (cond - neg) * scale
