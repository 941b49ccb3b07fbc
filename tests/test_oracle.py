"""Pins for the CPU oracle (oracle/denoise_oracle.py).

The reference ships no golden vectors for this path, so each oracle function is checked against
what the mathematics fixes: closed forms, special cases that reduce to a textbook formula, integer
brute force, and invariants chosen so that a plausible mistake (dropped term, wrong sign, wrong
half of a split, swapped chunk order, off-by-one position) fails.  All on small CPU shapes.
"""

from dataclasses import replace

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import denoise_oracle as O
from pi05_infer import synthetic as S

SMALL = S.ExpertGeometry(width=64, depth=2, num_heads=4, num_kv_heads=1, head_dim=16, mlp_dim=128,
                         action_dim=4, action_horizon=5)


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 numbers at |x| (8 significant bits)."""
    e = torch.floor(torch.log2(x.abs().clamp_min(1e-30)))
    return torch.pow(2.0, e - 7)


# ---------------------------------------------------------------------------- schedule / Euler


@pytest.mark.parametrize("n", [1, 2, 3, 5, 9, 10, 13, 16, 32])
def test_schedule_closed_form(n):
    ts = O.euler_timesteps(n)
    assert ts.dtype == torch.float32 and ts.shape == (n + 1,)
    assert ts[0].item() == 1.0 and ts[n].item() == 0.0
    assert ts[n - 1].item() == np.float32(1.0 / n)
    exact = torch.tensor([1.0 - i * (1.0 - 1.0 / n) / max(n - 1, 1) for i in range(n)], dtype=torch.float64)
    assert torch.all((ts[:n].double() - exact).abs() <= 4 * 2.0 ** -24)
    assert torch.all(ts[1:] < ts[:-1])  # strictly decreasing 1 -> 0


def test_schedule_ten_steps_matches_torch_linspace():
    # for N = 10 every torch linspace code path agrees (engine.py:425)
    ts = O.euler_timesteps(10)
    assert torch.equal(ts[:10], torch.linspace(1, 1 / 10, 10, dtype=torch.float32))


def test_euler_update_is_x_minus_v_delta():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 5, 4, generator=g)
    v = torch.randn(3, 5, 4, generator=g)
    ts = O.euler_timesteps(10)
    for s in range(10):
        t, d = ts[s], ts[s] - ts[s + 1]
        got = O.euler_update(x, v, t, d)
        # x0 (1 - (t - d)) + x1 (t - d) with x0 = x - v t, x1 = x + v (1 - t)  ==  x - v d
        torch.testing.assert_close(got, x - v * d, rtol=0, atol=4e-6)


def test_euler_constant_velocity_integrates_to_x_minus_v():
    x = torch.linspace(-2, 2, 20).reshape(1, 5, 4)
    v = torch.full_like(x, 0.75)
    ts = O.euler_timesteps(10)
    y = x.clone()
    for s in range(10):
        y = O.euler_update(y, v, ts[s], ts[s] - ts[s + 1])
    torch.testing.assert_close(y, x - v, rtol=0, atol=2e-6)


# ---------------------------------------------------------------------------- sinusoid / table


def test_sinusoid_special_values():
    emb0 = O.sinusoidal_time_embedding(torch.tensor([0.0]), 1024, 4e-3, 4.0)
    assert torch.equal(emb0[0, :512], torch.zeros(512)) and torch.equal(emb0[0, 512:], torch.ones(512))
    emb1 = O.sinusoidal_time_embedding(torch.tensor([1.0]), 1024, 4e-3, 4.0)[0]
    # last pair: period = max_period = 4 -> arg = 2*pi/4 = pi/2
    assert abs(emb1[511].item() - 1.0) < 1e-7 and abs(emb1[1023].item()) < 1e-7
    # first pair: period = min_period = 4e-3 -> arg = 500*pi
    assert abs(emb1[0].item()) < 1e-6 and abs(emb1[512].item() - 1.0) < 1e-7
    embh = O.sinusoidal_time_embedding(torch.tensor([0.5]), 1024, 4e-3, 4.0)[0]
    assert abs(embh[511].item() - 2 ** -0.5) < 1e-7 and abs(embh[1023].item() - 2 ** -0.5) < 1e-7
    for e in (emb1, embh):
        torch.testing.assert_close(e[:512] ** 2 + e[512:] ** 2, torch.ones(512), rtol=0, atol=1e-6)


def test_sinusoid_periods_are_geometric():
    # the frequency of pair i is 2*pi / (min * (max/min)^(i/511)); read it back from a tiny t
    t = 1e-7
    emb = O.sinusoidal_time_embedding(torch.tensor([t], dtype=torch.float64), 1024, 4e-3, 4.0)[0]
    freq = emb[:512].double() / t
    i = torch.arange(512, dtype=torch.float64)
    expect = 2 * np.pi / (4e-3 * (1000.0 ** (i / 511)))
    torch.testing.assert_close(freq, expect, rtol=1e-6, atol=0)


def test_table_zero_dense_weights_give_bias():
    g = SMALL
    w = S.make_weights(g)
    for wn, bn in O.norm_dense_names(O.geometry_from(g)):
        w[wn] = torch.zeros_like(w[wn])
    tab = O.adarms_table(w, O.geometry_from(g), 3)
    for n, (wn, bn) in enumerate(O.norm_dense_names(O.geometry_from(g))):
        for s in range(3):
            assert torch.equal(tab[s, n], w[bn])


def test_table_time_mlp_against_float64():
    g = SMALL
    og = O.geometry_from(g)
    w = S.make_weights(g)
    tab = O.adarms_table(w, og, 4)
    ts = O.euler_timesteps(4)
    wd = {k: v.double().numpy() for k, v in w.items() if v.dtype == torch.float32}
    silu = lambda z: z / (1 + np.exp(-z))
    for s in range(4):
        t = float(ts[s])
        i = np.arange(g.width // 2)
        period = 4e-3 * (4.0 / 4e-3) ** (i / (g.width // 2 - 1))
        arg = 2 * np.pi / period * t
        temb = np.concatenate([np.sin(arg), np.cos(arg)]).astype(np.float32).astype(np.float64)
        c = silu(wd["time_mlp_in.weight"] @ temb + wd["time_mlp_in.bias"])
        c = silu(wd["time_mlp_out.weight"] @ c + wd["time_mlp_out.bias"])
        for n, (wn, bn) in enumerate(O.norm_dense_names(og)):
            ref = wd[wn] @ c + wd[bn]
            np.testing.assert_allclose(tab[s, n].double().numpy(), ref, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------------- adaRMSNorm / residual


def _bf16_vals(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(torch.bfloat16).float()


def test_adarms_plain_rmsnorm_when_scale_shift_zero():
    W = 64
    h = _bf16_vals((3, 7, W), 1)
    mod = torch.zeros(3 * W)
    out, gate = O.ada_rms_norm(h, mod, 1e-6)
    ref = h.double() / torch.sqrt((h.double() ** 2).mean(-1, keepdim=True) + 1e-6)
    assert torch.all((out.double() - ref).abs() <= bf16_ulp(ref))
    assert torch.equal(gate, torch.zeros(W))


def test_adarms_chunk_order_scale_shift_gate():
    W = 64
    h = _bf16_vals((2, 5, W), 2)
    base, _ = O.ada_rms_norm(h, torch.zeros(3 * W), 1e-6)
    mod = torch.cat([torch.ones(W), torch.zeros(W), torch.full((W,), 0.3)])  # scale=1
    out, gate = O.ada_rms_norm(h, mod, 1e-6)
    torch.testing.assert_close(out, (base * 2).to(torch.bfloat16).float(), rtol=0, atol=0)
    assert torch.equal(gate, torch.full((W,), 0.3).to(torch.bfloat16).float())
    mod = torch.cat([torch.zeros(W), torch.full((W,), 0.5), torch.zeros(W)])  # shift=0.5
    out, _ = O.ada_rms_norm(h, mod, 1e-6)
    ref = h.double() / torch.sqrt((h.double() ** 2).mean(-1, keepdim=True) + 1e-6) + 0.5
    assert torch.all((out.double() - ref).abs() <= bf16_ulp(ref) * 1.01)


def test_gated_residual_gate_zero_and_one():
    x = _bf16_vals((4, 8), 3)
    y = _bf16_vals((4, 8), 4)
    assert torch.equal(O.gated_residual(x, y, torch.zeros(8)), x)
    assert torch.equal(O.gated_residual(x, y, torch.ones(8)), (x + y).to(torch.bfloat16).float())


# ---------------------------------------------------------------------------- RoPE


def test_rope_inv_freq_closed_form():
    inv = O.rope_inv_freq(256, 10000.0)
    assert inv[0].item() == 1.0
    assert abs(inv[64].item() - 0.01) <= 2 ** -24 * 0.01 * 2  # 10000^-0.5
    i = torch.arange(128, dtype=torch.float64)
    torch.testing.assert_close(inv.double(), 10000.0 ** (-i / 128), rtol=3e-7, atol=0)


def test_rope_position_zero_is_identity():
    pos = torch.zeros(1, 5, dtype=torch.int64)
    cos, sin = O.rope_cos_sin(pos, 16, 10000.0)
    assert torch.equal(cos, torch.ones_like(cos)) and torch.equal(sin, torch.zeros_like(sin))
    x = _bf16_vals((1, 5, 3, 16), 5)
    assert torch.equal(O.rope_apply(x, cos, sin), x)


def test_rope_is_complex_rotation_of_half_split_pairs():
    # rotate-half RoPE == multiplying z_d = x_d + i*x_{d+D/2} by exp(i*pos*inv_freq_d)
    D = 256
    pos = torch.tensor([[0, 3, 97, 968, 3321]], dtype=torch.int64)
    cos, sin = O.rope_cos_sin(pos, D, 10000.0)
    inv = O.rope_inv_freq(D, 10000.0).double().numpy()
    ang = pos[0].double().numpy()[:, None] * inv[None, :]
    assert np.all(np.abs(cos[0, :, :128].double().numpy() - np.cos(ang)) <= 2 ** -8)
    assert np.all(np.abs(sin[0, :, :128].double().numpy() - np.sin(ang)) <= 2 ** -8)
    assert torch.equal(cos[..., :128], cos[..., 128:]) and torch.equal(sin[..., :128], sin[..., 128:])
    x = _bf16_vals((1, 5, 2, D), 6)
    got = O.rope_apply(x, cos, sin).double().numpy()
    z = x[..., :128].double().numpy() + 1j * x[..., 128:].double().numpy()
    rot = z * (cos[..., :128].double().numpy() + 1j * sin[..., :128].double().numpy())[:, :, None, :]
    ref = np.concatenate([rot.real, rot.imag], axis=-1)
    tol = bf16_ulp(torch.from_numpy(ref)).numpy() + 1e-30
    assert np.all(np.abs(got - ref) <= tol)


# ---------------------------------------------------------------------------- positions / masks


def test_positions_and_mask_bruteforce():
    g = torch.Generator().manual_seed(7)
    B, P, A = 3, 17, 5
    pad = torch.rand(B, P, generator=g) > 0.3
    pad[:, 0] = True
    pos = O.position_ids(pad, A)
    mask = O.attention_mask_4d(pad, A)
    assert pos.dtype == torch.int64 and mask.dtype == torch.float32 and mask.shape == (B, 1, A, P + A)
    for b in range(B):
        n = sum(1 for p in range(P) if pad[b, p])
        for j in range(A):
            assert pos[b, j].item() == n + j
            for key in range(P + A):
                allowed = bool(pad[b, key]) if key < P else True
                assert mask[b, 0, j, key].item() == (0.0 if allowed else float(np.float32(O.MASK_MIN)))


# ---------------------------------------------------------------------------- attention / GeGLU


def test_mqa_attention_bruteforce():
    g = torch.Generator().manual_seed(8)
    B, H, A, S_, D = 2, 8, 5, 12, 16
    q = torch.randn(B, H, A, D, generator=g).to(torch.bfloat16).float()
    k = torch.randn(B, 1, S_, D, generator=g).to(torch.bfloat16).float()
    v = torch.randn(B, 1, S_, D, generator=g).to(torch.bfloat16).float()
    pad = torch.ones(B, S_ - A, dtype=torch.bool)
    pad[1, 3] = False
    pad[0, 0] = False
    mask = O.attention_mask_4d(pad, A)
    got = O.mqa_attention(q, k, v, mask, D ** -0.5)
    for b in range(B):
        for h in range(H):
            for a in range(A):
                keys = [j for j in range(S_) if mask[b, 0, a, j] == 0.0]
                sc = np.array([float(q[b, h, a].double() @ k[b, 0, j].double()) / np.sqrt(D) for j in keys])
                p = np.exp(sc - sc.max())
                p /= p.sum()
                o = sum(p[i] * v[b, 0, j].double().numpy() for i, j in enumerate(keys))
                row = got[b, a, h * D:(h + 1) * D].double().numpy()
                assert np.max(np.abs(row - o)) < 3e-2 * max(1.0, np.max(np.abs(o)))


def test_gelu_tanh_matches_library():
    x = torch.linspace(-8, 8, 10001)
    torch.testing.assert_close(O.gelu_tanh(x), F.gelu(x, approximate="tanh"), rtol=0, atol=2e-6)


def test_linear_bf16_rounds_the_exact_product():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(6, 64, generator=g).to(torch.bfloat16).float()
    w = torch.randn(32, 64, generator=g).to(torch.bfloat16).float()
    ref = x.double() @ w.double().T
    got = O.linear_bf16(x, w)
    assert torch.all((got.double() - ref).abs() <= bf16_ulp(ref) * 0.5 + 1e-6 * ref.abs() + 1e-30)


# ---------------------------------------------------------------------------- end-to-end special cases


def _small_inputs(g, P=9, B=1):
    k, v = S.make_prefix_kv(g, P, B)
    return k, v, S.full_prefix_pad(P, B), S.make_noise(g, B)


def test_zero_gates_make_expert_the_final_norm_of_the_embedding():
    g = SMALL
    og = O.geometry_from(g)
    w = S.zero_gate_weights(S.make_weights(g), g)
    k, v, pad, x = _small_inputs(g)
    tab = O.adarms_table(w, og, 2)
    st = O.prepare_state(og, k, v, pad)
    vel = O.velocity(w, og, x, tab[0], st)
    h = (x @ w["action_in_proj.weight"].T + w["action_in_proj.bias"]).to(torch.bfloat16).float()
    n, _ = O.ada_rms_norm(h, tab[0, og.num_norms - 1], og.rms_eps)
    ref = n @ w["action_out_proj.weight"].T + w["action_out_proj.bias"]
    torch.testing.assert_close(vel, ref, rtol=0, atol=0)


def test_constant_velocity_loop_closed_form():
    g = SMALL
    og = O.geometry_from(g)
    w = S.zero_gate_weights(S.make_weights(g), g)
    w["action_out_proj.weight"] = torch.zeros_like(w["action_out_proj.weight"])
    w["action_out_proj.bias"] = torch.full_like(w["action_out_proj.bias"], 0.25)
    k, v, pad, x = _small_inputs(g)
    act, vs = O.sample_actions(w, og, k, v, pad, x, 10)
    assert torch.equal(vs, torch.full_like(vs, 0.25))
    torch.testing.assert_close(act, x - 0.25, rtol=0, atol=2e-6)


def test_kv_cache_tail_holds_rotated_suffix_keys():
    # the static cache row P + t must hold rope(k_t) and raw v_t (modeling_gemma.py:418-427)
    g = SMALL
    og = O.geometry_from(g)
    w = S.make_weights(g)
    k, v, pad, x = _small_inputs(g, P=7)
    tab = O.adarms_table(w, og, 1)
    st = O.prepare_state(og, k, v, pad)
    O.velocity(w, og, x, tab[0], st)
    assert torch.equal(st.k_cache[0][:, 0, :7], k[:, 0].float())
    assert torch.all(st.k_cache[0][:, 0, 7:].abs().sum(-1) > 0)
    assert torch.all(st.v_cache[0][:, 0, 7:].abs().sum(-1) > 0)


# ---------------------------------------------------------------------------- layer composition
#
# GemmaDecoderLayer (modeling_gemma.py:486-517): the input norm takes mod[0] and its gate scales
# the attention branch; the post-attention norm takes mod[1] and its gate scales the MLP branch;
# GemmaModel hands layer i the slices 2i, 2i+1 and the final norm slice 2L
# (modeling_gemma.py:773, 782-783).  Each branch is isolated by zeroing the other branch's output
# projection, and checked against a reference assembled here from library routines
# (F.rms_norm, F.gelu, F.scaled_dot_product_attention, RoPE as a complex rotation); the
# variants with the slices or the gates swapped must fail the same check.


def _distinct_mods(W, seed=11):
    """Two modulation rows with clearly different scale / shift / gate per norm."""
    g = torch.Generator().manual_seed(seed)
    r = lambda: 0.1 * torch.randn(W, generator=g)
    mod_a = torch.cat([0.5 + r(), 0.3 + r(), 0.8 + r()])
    mod_b = torch.cat([-0.4 + r(), -0.2 + r(), 1.5 + r()])
    return torch.stack([mod_a, mod_b])


def _lib_norm(h, mod, eps):
    W = h.shape[-1]
    scale, shift, gate = mod[:W], mod[W:2 * W], mod[2 * W:]
    n = F.rms_norm(h, (W,), eps=eps) * (1 + scale) + shift
    return n.to(torch.bfloat16).float(), gate.to(torch.bfloat16).float()


def _bf(x):
    return x.to(torch.bfloat16).float()


def _lib_rope(x, pos, theta):
    """x [B, A, H, D]; rotation of (x[d], x[d + D/2]) by pos * theta^(-2d/D), in float64."""
    D = x.shape[-1]
    inv = theta ** (-torch.arange(0, D, 2, dtype=torch.float64) / D)
    ang = pos.double()[:, :, None, None] * inv
    z = torch.complex(x[..., : D // 2].double(), x[..., D // 2:].double()) * torch.polar(torch.ones_like(ang), ang)
    return _bf(torch.cat([z.real, z.imag], dim=-1).float())


def _lib_attention_branch(w, g, i, h, mod, k_pre, v_pre, pad):
    """bf16(h + bf16(o_proj(attention(norm(h; mod))) * gate)), library attention in fp32."""
    p = f"{O.EXPERT_PREFIX}layers.{i}."
    B, A, _ = h.shape
    H, D = g.num_heads, g.head_dim
    n, gate = _lib_norm(h, mod, g.rms_eps)
    q = _bf(n @ w[p + "self_attn.q_proj.weight"].float().T).reshape(B, A, H, D)
    k = _bf(n @ w[p + "self_attn.k_proj.weight"].float().T).reshape(B, A, 1, D)
    v = _bf(n @ w[p + "self_attn.v_proj.weight"].float().T).reshape(B, A, 1, D)
    pos = pad.sum(-1, keepdim=True) + torch.arange(A)[None, :]
    q, k = _lib_rope(q, pos, g.rope_theta), _lib_rope(k, pos, g.rope_theta)
    K = torch.cat([k_pre[:, i].float(), k[:, :, 0]], dim=1)[:, None]  # [B, 1, P + A, D]
    V = torch.cat([v_pre[:, i].float(), v[:, :, 0]], dim=1)[:, None]
    allowed = torch.cat([pad, torch.ones(B, A, dtype=torch.bool)], dim=1)[:, None, None, :]
    o = F.scaled_dot_product_attention(q.transpose(1, 2), K.expand(B, H, -1, -1), V.expand(B, H, -1, -1), attn_mask=allowed)
    o = _bf(o).transpose(1, 2).reshape(B, A, H * D)
    y = _bf(o @ w[p + "self_attn.o_proj.weight"].float().T)
    return _bf(h + _bf(y * gate))


def _lib_mlp_branch(w, g, i, h, mod):
    """bf16(h + bf16(down(bf16(gelu_tanh(bf16(gate_proj(n))) * up_proj(n))) * gate)), n = norm(h; mod)."""
    p = f"{O.EXPERT_PREFIX}layers.{i}."
    n, gate = _lib_norm(h, mod, g.rms_eps)
    gt = _bf(n @ w[p + "mlp.gate_proj.weight"].float().T)
    up = n @ w[p + "mlp.up_proj.weight"].float().T
    act = _bf(F.gelu(gt, approximate="tanh") * up)
    y = _bf(act @ w[p + "mlp.down_proj.weight"].float().T)
    return _bf(h + _bf(y * gate))


def _lib_layer(w, g, i, h, mod2, k_pre, v_pre, pad):
    return _lib_mlp_branch(w, g, i, _lib_attention_branch(w, g, i, h, mod2[0], k_pre, v_pre, pad), mod2[1])


def _agree(got, ref, h):
    """Cosine and relative max error of the branch contributions (got - h) vs (ref - h)."""
    a, b = (got - h).double().flatten(), (ref - h).double().flatten()
    cos = F.cosine_similarity(a, b, dim=0).item()
    rel = ((a - b).abs().max() / b.abs().max()).item()
    return cos, rel


def _layer_case(P=7, seed=3):
    g = SMALL
    og = O.geometry_from(g)
    # weights large enough that each branch's contribution is not lost in the bf16 residual add
    w = S.make_weights(g, seed=seed, std=0.15)
    k, v, _, x = _small_inputs(g, P=P)
    pad = torch.ones(1, P, dtype=torch.bool)
    pad[0, 2] = False  # one padded prefix key
    h = _bf(0.1 * torch.randn(1, g.action_horizon, g.width, generator=torch.Generator().manual_seed(seed)))
    return g, og, w, k, v, pad, h


def test_expert_layer_mlp_branch_uses_second_slice_and_gate():
    g, og, w, k, v, pad, h = _layer_case()
    p = f"{O.EXPERT_PREFIX}layers.0."
    w[p + "self_attn.o_proj.weight"] = torch.zeros_like(w[p + "self_attn.o_proj.weight"])  # attention adds 0
    mod2 = _distinct_mods(g.width)
    st = O.prepare_state(og, k, v, pad)
    got = O.expert_layer(w, og, 0, h, mod2, st)
    cos, rel = _agree(got, _lib_mlp_branch(w, g, 0, h, mod2[1]), h)
    assert cos >= 0.9999 and rel <= 2e-2, (cos, rel)
    # the MLP norm fed the first slice, or the MLP scaled by the attention gate, must fail
    swapped = torch.stack([mod2[0], mod2[0]])
    gate_swapped = mod2[1].clone()
    gate_swapped[2 * g.width:] = mod2[0, 2 * g.width:]
    for bad in (_lib_mlp_branch(w, g, 0, h, swapped[1]), _lib_mlp_branch(w, g, 0, h, gate_swapped)):
        cos_b, rel_b = _agree(got, bad, h)
        assert cos_b < 0.999 or rel_b > 0.1, (cos_b, rel_b)


def test_expert_layer_attention_branch_uses_first_slice_and_gate():
    g, og, w, k, v, pad, h = _layer_case()
    p = f"{O.EXPERT_PREFIX}layers.0."
    w[p + "mlp.down_proj.weight"] = torch.zeros_like(w[p + "mlp.down_proj.weight"])  # MLP adds 0
    mod2 = _distinct_mods(g.width)
    st = O.prepare_state(og, k, v, pad)
    got = O.expert_layer(w, og, 0, h, mod2, st)
    cos, rel = _agree(got, _lib_attention_branch(w, g, 0, h, mod2[0], k, v, pad), h)
    assert cos >= 0.9999 and rel <= 2e-2, (cos, rel)
    gate_swapped = mod2[0].clone()
    gate_swapped[2 * g.width:] = mod2[1, 2 * g.width:]
    for bad in (_lib_attention_branch(w, g, 0, h, mod2[1], k, v, pad), _lib_attention_branch(w, g, 0, h, gate_swapped, k, v, pad)):
        cos_b, rel_b = _agree(got, bad, h)
        assert cos_b < 0.999 or rel_b > 0.1, (cos_b, rel_b)


def test_velocity_feeds_layer_i_slices_2i_2i1_and_final_norm_2L():
    g = SMALL  # depth 2: norms 0..4
    og = O.geometry_from(g)
    w = S.make_weights(g, seed=5, std=0.15)
    k, v, _, x = _small_inputs(g, P=6)
    pad = torch.ones(1, 6, dtype=torch.bool)
    gen = torch.Generator().manual_seed(12)
    mod = torch.stack([torch.cat([(-1) ** j * 0.3 * (j + 1) + 0.1 * torch.randn(g.width, generator=gen),
                                  0.1 * (j - 2) + 0.1 * torch.randn(g.width, generator=gen),
                                  0.4 + 0.3 * j + 0.1 * torch.randn(g.width, generator=gen)]) for j in range(og.num_norms)])
    st = O.prepare_state(og, k, v, pad)
    got = O.velocity(w, og, x, mod, st)

    def lib_velocity(slices, final):
        h = _bf(x @ w["action_in_proj.weight"].T + w["action_in_proj.bias"])
        for i in range(g.depth):
            h = _lib_layer(w, g, i, h, mod[list(slices(i))], k, v, pad)
        n, _ = _lib_norm(h, mod[final], g.rms_eps)
        return n @ w["action_out_proj.weight"].T + w["action_out_proj.bias"]

    ref = lib_velocity(lambda i: (2 * i, 2 * i + 1), 2 * g.depth)
    cos = F.cosine_similarity(got.double().flatten(), ref.double().flatten(), dim=0).item()
    rel = ((got - ref).abs().max() / ref.abs().max()).item()
    assert cos >= 0.9999 and rel <= 2e-2, (cos, rel)
    for slices, final in (((lambda i: (i, i + 1)), 2 * g.depth), ((lambda i: (2 * i + 1, 2 * i)), 2 * g.depth),
                          ((lambda i: (2 * i, 2 * i + 1)), 0)):
        bad = lib_velocity(slices, final)
        cos_b = F.cosine_similarity(got.double().flatten(), bad.double().flatten(), dim=0).item()
        rel_b = ((got - bad).abs().max() / bad.abs().max()).item()
        assert cos_b < 0.999 or rel_b > 0.1, (cos_b, rel_b)
