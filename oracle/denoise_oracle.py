"""CPU oracle of the pi0.5 action-expert denoise loop.

TEST INFRASTRUCTURE ONLY.  This module is the checker: ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it; the product
(``pi05-infer_amd/``) never does, and it is never the thing measured on the GPU.

It restates the reference's eager fp32/bf16 arithmetic in PyTorch on the CPU, in fp32, with an
explicit bf16 rounding (``_bf``) at every point where the reference holds a bf16 tensor.  Each
function cites the reference lines it follows (paths relative to the pi05-infer repository).

Rounding ledger of one step (what this oracle encodes):

* ``action_in_proj`` fp32 -> bf16 (modeling_gemma.py:724-725);
* adaRMSNorm: fp32 statistics and modulation, output and gate rounded to bf16
  (modeling_gemma.py:82-116);
* QKV GEMM rounded to bf16, RoPE in fp32 from the bf16 GEMM values and bf16 cos/sin, rounded
  once (the shipped fused kernel, rlinf_fused_denoise.py:264-278); v is the bf16 GEMM value;
* scores bf16(q.k^T), scaled by 1/16 in bf16, + fp32 mask, fp32 softmax, P rounded to bf16,
  O = bf16(P.V) (modeling_gemma.py:252-275);
* o_proj / down_proj outputs bf16; gated residual ``x + y*gate`` in eager bf16 semantics, i.e.
  ``bf16(x + bf16(y*gate))`` (modeling_gemma.py:231-249);
* GeGLU as the shipped fused kernel defines it: bf16(gelu_tanh(bf16(g)) * u) with ``u`` the fp32
  accumulator (rlinf_fused_denoise.py:166-173);
* final norm bf16 -> fp32 -> ``action_out_proj`` fp32 (engine.py:754-767);
* Euler flow_ode update in fp32 in the reference's op order (engine.py:664-675).

The adaRMS modulation table, the timestep schedule and the sinusoid are fp32/f64 exactly as in
engine.py:411-429, 578-599 and pi0_pytorch.py:29-46, 296-334.  The reference runs its fp32
linears in TF32 on NVIDIA (pi0_pytorch.py:115); this oracle uses full fp32, which is the same
code's CPU semantics.

Pins (see tests/test_oracle.py): closed forms (schedule, sinusoid, Euler algebra), textbook
identities (RMSNorm, RoPE norm preservation and position 0, softmax attention by brute force,
MQA = repeat_kv), special cases (zero dense weights => mod = bias; zero gates => identity
layers), integer brute force for positions and masks.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch
import torch.nn.functional as F

F32 = torch.float32
BF16 = torch.bfloat16

EXPERT_PREFIX = "paligemma_with_expert.gemma_expert.model."
MASK_MIN = -2.3819763e38  # pi0_pytorch.py:163


def _bf(x: torch.Tensor) -> torch.Tensor:
    """Round to bf16 (round-to-nearest-even) and return as fp32."""
    return x.to(BF16).to(F32)


@dataclass
class OracleGeometry:
    width: int = 1024
    depth: int = 18
    num_heads: int = 8
    num_kv_heads: int = 1
    head_dim: int = 256
    mlp_dim: int = 4096
    action_dim: int = 32
    action_horizon: int = 50
    rms_eps: float = 1e-6
    rope_theta: float = 10000.0
    time_min_period: float = 4e-3
    time_max_period: float = 4.0

    @property
    def num_norms(self) -> int:
        return 2 * self.depth + 1


# --------------------------------------------------------------------------------------------
# schedule, sinusoid, modulation table
# --------------------------------------------------------------------------------------------


def linspace_gpu(start: float, end: float, steps: int, dtype=np.float32) -> torch.Tensor:
    """``torch.linspace`` as its elementwise GPU kernel evaluates it: with
    ``step = (end - start) / (steps - 1)``, element ``i`` is ``start + step*i`` for
    ``i < steps // 2`` and ``end - step*(steps - i - 1)`` otherwise, every op in ``dtype``.

    The reference builds its schedules on its CUDA device; torch's CPU linspace uses a vectorised
    ``arange`` for part of the range and rounds differently for many ``steps`` (not for 10)."""
    if steps == 1:
        return torch.from_numpy(np.array([start], dtype=dtype))
    s = dtype(start)
    e = dtype(end)
    step = dtype((e - s) / dtype(steps - 1))
    half = steps // 2
    vals = [s + step * dtype(i) if i < half else e - step * dtype(steps - i - 1) for i in range(steps)]
    return torch.from_numpy(np.array(vals, dtype=dtype))


def euler_timesteps(num_steps: int) -> torch.Tensor:
    """``linspace(1, 1/N, N) ++ [0]`` in fp32 (engine.py:411-429)."""
    ts = linspace_gpu(1.0, 1 / num_steps, num_steps)
    return torch.cat([ts, torch.zeros(1, dtype=F32)])


def sinusoidal_time_embedding(t: torch.Tensor, dim: int, min_period: float, max_period: float) -> torch.Tensor:
    """pi0_pytorch.py:29-46 (float64 on device, ``get_safe_dtype``), cast to ``t.dtype`` (line 300)."""
    if dim % 2:
        raise ValueError("dimension must be even")
    fraction = linspace_gpu(0.0, 1.0, dim // 2, np.float64)
    period = min_period * (max_period / min_period) ** fraction
    scaling_factor = 1.0 / period * 2 * math.pi
    sin_input = scaling_factor[None, :] * t[:, None]
    return torch.cat([torch.sin(sin_input), torch.cos(sin_input)], dim=1).to(t.dtype)


def norm_dense_names(g: OracleGeometry) -> list[tuple[str, str]]:
    """adaRMS dense (weight, bias) names in the order the table stacks them (engine.py:580-586)."""
    names = []
    for i in range(g.depth):
        p = f"{EXPERT_PREFIX}layers.{i}."
        names.append((p + "input_layernorm.dense.weight", p + "input_layernorm.dense.bias"))
        names.append((p + "post_attention_layernorm.dense.weight", p + "post_attention_layernorm.dense.bias"))
    names.append((EXPERT_PREFIX + "norm.dense.weight", EXPERT_PREFIX + "norm.dense.bias"))
    return names


def time_condition(w: dict, g: OracleGeometry, t: torch.Tensor) -> torch.Tensor:
    """adaRMS condition: silu(time_mlp_out(silu(time_mlp_in(sinusoid(t))))) (pi0_pytorch.py:296-334)."""
    temb = sinusoidal_time_embedding(t, g.width, g.time_min_period, g.time_max_period)
    x = F.linear(temb, w["time_mlp_in.weight"].float(), w["time_mlp_in.bias"].float())
    x = F.silu(x)
    x = F.linear(x, w["time_mlp_out.weight"].float(), w["time_mlp_out.bias"].float())
    return F.silu(x)


def adarms_table(w: dict, g: OracleGeometry, num_steps: int) -> torch.Tensor:
    """Modulation table ``[num_steps, 2L+1, 3W]`` fp32 (engine.py:578-599, batch row 0)."""
    ts = euler_timesteps(num_steps)
    names = norm_dense_names(g)
    rows = []
    for s in range(num_steps):
        cond = time_condition(w, g, ts[s].reshape(1))
        rows.append(torch.stack([F.linear(cond, w[wn].float(), w[bn].float())[0] for wn, bn in names]))
    return torch.stack(rows)


# --------------------------------------------------------------------------------------------
# step invariants: positions, masks, rotary tables
# --------------------------------------------------------------------------------------------


def make_att_2d_masks(pad_masks: torch.Tensor, att_masks: torch.Tensor) -> torch.Tensor:
    """pi0_pytorch.py:56-85."""
    cumsum = torch.cumsum(att_masks, dim=1)
    att_2d = cumsum[:, None, :] <= cumsum[:, :, None]
    pad_2d = pad_masks[:, None, :] * pad_masks[:, :, None]
    return att_2d & pad_2d


def suffix_masks(batch: int, horizon: int) -> tuple[torch.Tensor, torch.Tensor]:
    """pi0.5 suffix pad (all ones) and att masks ``[1] + [0]*(A-1)`` (pi0_pytorch.py:339-349)."""
    pad = torch.ones(batch, horizon, dtype=torch.bool)
    att = torch.tensor([1] + [0] * (horizon - 1), dtype=F32)[None, :].expand(batch, horizon)
    return pad, att


def position_ids(prefix_pad: torch.Tensor, horizon: int) -> torch.Tensor:
    """``sum(prefix_pad) + cumsum(suffix_pad) - 1`` int64 ``[B, A]`` (engine.py:476-477)."""
    pad, _ = suffix_masks(prefix_pad.shape[0], horizon)
    offsets = torch.sum(prefix_pad, dim=-1)[:, None]
    return offsets + torch.cumsum(pad, dim=1) - 1


def attention_mask_4d(prefix_pad: torch.Tensor, horizon: int) -> torch.Tensor:
    """Additive fp32 mask ``[B, 1, A, P+A]`` (engine.py:471-478; pi0_pytorch.py:160-163)."""
    b, p = prefix_pad.shape
    pad, att = suffix_masks(b, horizon)
    prefix_2d = prefix_pad[:, None, :].expand(b, horizon, p)
    suffix_2d = make_att_2d_masks(pad, att)
    full = torch.cat([prefix_2d, suffix_2d], dim=2)
    return torch.where(full[:, None, :, :], 0.0, MASK_MIN)


def rope_inv_freq(head_dim: int, theta: float) -> torch.Tensor:
    """transformers' default RoPE init: ``1 / theta ** (arange(0, D, 2) / D)`` in fp32."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).to(F32) / head_dim))


def rope_cos_sin(pos: torch.Tensor, head_dim: int, theta: float) -> tuple[torch.Tensor, torch.Tensor]:
    """Rotary cos/sin ``[B, A, D]`` rounded to bf16, returned as fp32 (modeling_gemma.py:169-182)."""
    inv = rope_inv_freq(head_dim, theta)
    b = pos.shape[0]
    inv_e = inv[None, :, None].float().expand(b, -1, 1)
    pos_e = pos[:, None, :].float()
    freqs = (inv_e @ pos_e).transpose(1, 2)
    emb = torch.cat((freqs, freqs), dim=-1)
    return _bf(emb.cos()), _bf(emb.sin())


# --------------------------------------------------------------------------------------------
# expert layer pieces
# --------------------------------------------------------------------------------------------


def ada_rms_norm(h: torch.Tensor, mod: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """adaRMSNorm with a precomputed modulation (modeling_gemma.py:82-116).

    ``h`` holds bf16 values (fp32 storage) ``[..., W]``; ``mod`` is fp32 ``[3W]`` (scale, shift,
    gate in that order, line 111).  Returns (bf16 output, bf16 gate).
    """
    var = torch.mean(torch.square(h), dim=-1, keepdim=True)
    normed = h * torch.rsqrt(var + eps)
    scale, shift, gate = torch.chunk(mod, 3, dim=-1)
    out = normed * (1 + scale) + shift
    return _bf(out), _bf(gate)


def gated_residual(x: torch.Tensor, y: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """``x + y * gate`` on bf16 tensors, eager semantics (modeling_gemma.py:231-249)."""
    return _bf(x + _bf(y * gate))


def linear_bf16(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """bf16 ``nn.Linear`` without bias: fp32 accumulation, bf16 output."""
    return _bf(x @ w.T)


def rope_apply(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE as the fused QKV kernel computes it (rlinf_fused_denoise.py:264-278).

    ``x`` ``[B, A, H, D]`` bf16 values, ``cos``/``sin`` ``[B, A, D]`` bf16 values; fp32 math,
    one bf16 rounding.  ``(x*cos) + (rotate_half(x)*sin)`` with ``rotate_half(x) = cat(-x_hi, x_lo)``
    (modeling_gemma.py:185-216).
    """
    half = x.shape[-1] // 2
    c = cos[:, :, None, :]
    s = sin[:, :, None, :]
    lo, hi = x[..., :half], x[..., half:]
    o_lo = lo * c[..., :half] - hi * s[..., :half]
    o_hi = hi * c[..., half:] + lo * s[..., half:]
    return _bf(torch.cat([o_lo, o_hi], dim=-1))


def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    """GELU, tanh approximation, in the fused kernel's op order (rlinf_fused_denoise.py:168-173)."""
    t3 = x * 0.5
    t5 = (x * x) * x
    t8 = x + t5 * 0.044715
    t11 = torch.tanh(t8 * 0.7978845608028654)
    return t3 * (t11 + 1.0)


def mqa_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask4d: torch.Tensor, scaling: float) -> torch.Tensor:
    """Eager attention with ``repeat_kv`` (modeling_gemma.py:219-228, 252-275).

    ``q`` ``[B, H, A, D]``, ``k``/``v`` ``[B, Hkv, S, D]`` (bf16 values), ``mask4d`` fp32 ``[B,1,A,S]``.
    Returns ``[B, A, H*D]`` bf16 values.
    """
    b, h, a, d = q.shape
    n_rep = h // k.shape[1]
    kr = k[:, :, None].expand(b, k.shape[1], n_rep, k.shape[2], d).reshape(b, h, k.shape[2], d)
    vr = v[:, :, None].expand(b, v.shape[1], n_rep, v.shape[2], d).reshape(b, h, v.shape[2], d)
    scores = _bf(q @ kr.transpose(2, 3))
    scores = _bf(scores * scaling)
    scores = scores + mask4d[:, :, :, : kr.shape[-2]]
    p = _bf(torch.softmax(scores, dim=-1, dtype=F32))
    o = _bf(p @ vr)
    return o.transpose(1, 2).reshape(b, a, h * d)


@dataclass
class StepState:
    """Per-predict invariants (engine.py:453-524) + the static KV cache (modeling_gemma.py:312-329)."""

    mask4d: torch.Tensor
    pos: torch.Tensor
    cos: torch.Tensor
    sin: torch.Tensor
    k_cache: list  # per layer [B, 1, P+A, D] fp32 holding bf16 values
    v_cache: list
    prefix_len: int
    trace: dict = field(default_factory=dict)


def expert_layer(w: dict, g: OracleGeometry, i: int, h: torch.Tensor, mod2: torch.Tensor, st: StepState) -> torch.Tensor:
    """GemmaDecoderLayer.forward on the fused denoise path (modeling_gemma.py:460-517, 370-397)."""
    p = f"{EXPERT_PREFIX}layers.{i}."
    b, a, _ = h.shape
    H, D, Hkv = g.num_heads, g.head_dim, g.num_kv_heads
    n1, gate1 = ada_rms_norm(h, mod2[0], g.rms_eps)
    wq = w[p + "self_attn.q_proj.weight"].float()
    wk = w[p + "self_attn.k_proj.weight"].float()
    wv = w[p + "self_attn.v_proj.weight"].float()
    wqkv = torch.cat([wq, wk, wv], dim=0)  # build_qkv_fused, modeling_gemma.py:345
    qkv = linear_bf16(n1, wqkv)
    q = qkv[..., : H * D].reshape(b, a, H, D)
    k = qkv[..., H * D : (H + Hkv) * D].reshape(b, a, Hkv, D)
    v = qkv[..., (H + Hkv) * D :].reshape(b, a, Hkv, D)
    q = rope_apply(q, st.cos, st.sin)
    k = rope_apply(k, st.cos, st.sin)
    P = st.prefix_len
    st.k_cache[i][:, :, P:, :] = k.transpose(1, 2)
    st.v_cache[i][:, :, P:, :] = v.transpose(1, 2)
    o = mqa_attention(q.transpose(1, 2), st.k_cache[i], st.v_cache[i], st.mask4d, D ** -0.5)
    y = linear_bf16(o, w[p + "self_attn.o_proj.weight"].float())
    h = gated_residual(h, y, gate1)
    n2, gate2 = ada_rms_norm(h, mod2[1], g.rms_eps)
    gte = linear_bf16(n2, w[p + "mlp.gate_proj.weight"].float())
    up = n2 @ w[p + "mlp.up_proj.weight"].float().T
    act = _bf(gelu_tanh(gte) * up)
    y = linear_bf16(act, w[p + "mlp.down_proj.weight"].float())
    return gated_residual(h, y, gate2)


def velocity(w: dict, g: OracleGeometry, x_t: torch.Tensor, mod: torch.Tensor, st: StepState) -> torch.Tensor:
    """get_velocity: embed_suffix (action_in_proj) -> expert -> final norm -> action_out_proj
    (engine.py:681-768; pi0_pytorch.py:303-306; modeling_gemma.py:722-783)."""
    emb = F.linear(x_t, w["action_in_proj.weight"].float(), w["action_in_proj.bias"].float())
    h = _bf(emb)
    for i in range(g.depth):
        h = expert_layer(w, g, i, h, mod[2 * i : 2 * i + 2], st)
    out, _ = ada_rms_norm(h, mod[g.num_norms - 1], g.rms_eps)
    return F.linear(out, w["action_out_proj.weight"].float(), w["action_out_proj.bias"].float())


def euler_update(x_t: torch.Tensor, v_t: torch.Tensor, t: torch.Tensor, delta: torch.Tensor) -> torch.Tensor:
    """flow_ode mean, fp32, reference op order (engine.py:664-675)."""
    x0_pred = x_t - v_t * t
    x1_pred = x_t + v_t * (1 - t)
    x0_weight = 1 - (t - delta)
    x1_weight = t - delta
    return x0_pred * x0_weight + x1_pred * x1_weight


def prepare_state(g: OracleGeometry, k_prefix: torch.Tensor, v_prefix: torch.Tensor, prefix_pad: torch.Tensor) -> StepState:
    """Static KV priming + hoisted invariants. ``k_prefix``/``v_prefix`` are bf16 ``[B, L, P, D]``."""
    b, L, P, D = k_prefix.shape
    a = g.action_horizon
    pos = position_ids(prefix_pad, a)
    cos, sin = rope_cos_sin(pos, D, g.rope_theta)
    kc, vc = [], []
    for i in range(L):
        kb = torch.zeros(b, 1, P + a, D, dtype=F32)
        vb = torch.zeros(b, 1, P + a, D, dtype=F32)
        kb[:, 0, :P] = k_prefix[:, i].float()
        vb[:, 0, :P] = v_prefix[:, i].float()
        kc.append(kb)
        vc.append(vb)
    return StepState(attention_mask_4d(prefix_pad, a), pos, cos, sin, kc, vc, P)


def sample_actions(w: dict, g: OracleGeometry, k_prefix: torch.Tensor, v_prefix: torch.Tensor,
                   prefix_pad: torch.Tensor, noise: torch.Tensor, num_steps: int = 10,
                   table: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """The denoise loop of sample_actions (engine.py:344-406, eager branch, noise given).

    Returns (actions ``[B, A, a]``, per-step velocities ``[num_steps, B, A, a]``), fp32.
    """
    if table is None:
        table = adarms_table(w, g, num_steps)
    st = prepare_state(g, k_prefix, v_prefix, prefix_pad)
    ts = euler_timesteps(num_steps)
    x = noise.to(F32)
    vs = []
    for s in range(num_steps):
        v = velocity(w, g, x, table[s], st)
        t = ts[s]
        delta = ts[s] - ts[s + 1]
        x = euler_update(x, v, t, delta)
        vs.append(v)
    return x, torch.stack(vs)


def geometry_from(obj) -> OracleGeometry:
    """Oracle geometry from any object with the same field names."""
    return OracleGeometry(**{f: getattr(obj, f) for f in OracleGeometry.__dataclass_fields__})
