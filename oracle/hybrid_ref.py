"""The hybrid models' per-token mixers, routers and experts (CPU torch).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Two arithmetic policies, each the one the reference states for its model:

* **C4, Qwen3.5-35B-A3B** -- the example's plain-torch twin
  ``examples/qwen3_5_35b_a3b-tilelang/kernels/torch_ref.py`` (its "dtype policy",
  ``:22-40``): activations and state f32; a matmul runs at the weights' dtype, so
  the activation is cast to bf16, the product summed in f32 and rounded to bf16
  once, and handed on as f32 (``_mm``/``_wm`` ``:134-143``); everything else in
  f32.  The GDN recurrent state is f32 (the benchmark's "fp32 recurrent state").
* **C5, Granite-4.0-H** -- the authored HIR
  ``examples/granite_4_0_h_small-cuda/model.py``: bf16 activations, every binary
  op rounded to bf16 (binary ops never promote, ``ir/hir/math/binary.py:130-139``),
  the explicit f32 casts where the HIR writes them, f32 SSM state.  Weights are
  fp8-e4m3fn with one f32 scale per output channel (the benchmark's C5; the
  reference has no fp8 GEMV, so the build defines ``W = f32(e4m3) * scale[out]``
  with f32 accumulation -- parity there is against that definition).

Every function cites the reference function it restates.  Matmul sums run in f64
(``exact=True``) or f32; the kernels' f32 sums differ only in order.
"""
from __future__ import annotations

from contextlib import contextmanager

import torch

F32, BF16 = torch.float32, torch.bfloat16

_ROUND = True


def bf(x: torch.Tensor) -> torch.Tensor:
    """Round to bf16 and hand back as f32 (inside ``unrounded()``: f32 as is)."""
    return x.to(BF16).float() if _ROUND else x.float()


@contextmanager
def unrounded():
    """Every bf16 rounding point of this module becomes the identity: the oracle
    is then the models' f32 mathematics, the form an independent f32
    implementation (Hugging Face's modules) is compared with to pin how the
    whole steps compose their pieces."""
    global _ROUND
    old, _ROUND = _ROUND, False
    try:
        yield
    finally:
        _ROUND = old


def mm_rows(w: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """sum_k w[n][k] x[..., k] in f64, as f32 (w [N][K] (out, in), x [..., K])."""
    return (x.double() @ w.double().t()).float()


# ---------------------------------------------------------------------------
# fp8-e4m3fn weights with per-output-channel scales (a23)
# ---------------------------------------------------------------------------
def fp8_dequant(codes: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """``W = f32(e4m3fn(code)) * scale[out]``: codes uint8 [N][K], scale f32 [N].
    Every e4m3fn value is exact in f32 (``torch.float8_e4m3fn -> float32``)."""
    return codes.view(torch.float8_e4m3fn).float() * scale.float()[:, None]


def gemv_fp8(codes: torch.Tensor, scale: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """bf16 activations x [B][K] against fp8 rows: y[b][n] = scale[n] *
    sum_k e4m3(w[n][k]) * x[b][k], f32 (the build's definition; see the header)."""
    raw = codes.view(torch.float8_e4m3fn).double()
    return ((x.double() @ raw.t()) * scale.double()[None, :]).float()


# ---------------------------------------------------------------------------
# Routers (a17, a21)
# ---------------------------------------------------------------------------
def topk_ordered(v: torch.Tensor, k: int):
    """``torch.topk(v, k)`` with its tie order fixed: largest first, equal values
    by ascending index.  torch.topk leaves the order of equal values unspecified
    (its CPU and GPU kernels differ), and bf16-valued router logits tie often
    (256 experts, 8 mantissa bits); the build's routers use this order."""
    vals, idx = torch.sort(v, dim=-1, descending=True, stable=True)
    return vals[..., :k], idx[..., :k]


def route_softmax_topk(logits: torch.Tensor, k: int):
    """Qwen3.5 router after its projection (torch_ref.py:417-430, HF
    ``Qwen3_5MoeTopKRouter``): softmax over every expert in f32, the top k
    (largest first, ties to the lower index), renormalised by their sum.
    -> (weights f32 [B][k], indices i64 [B][k])."""
    probs = torch.softmax(logits.float(), dim=-1)
    vals, idx = topk_ordered(probs, k)
    return vals / vals.sum(dim=-1, keepdim=True), idx


def route_topk_softmax(logits: torch.Tensor, k: int):
    """Granite router after its projection (model.py:376-390, HF
    ``GraniteMoeHybridTopKRouter``): the top k logits (f32, ties to the lower
    index), then a softmax over those k alone, cast to the activation dtype.
    -> (weights as bf16 values in f32 [B][k], indices i64 [B][k])."""
    vals, idx = topk_ordered(logits.float(), k)
    return bf(torch.softmax(vals, dim=-1)), idx


def _over_set(scores: torch.Tensor, idx: torch.Tensor):
    """The entries of *scores* [B][E] at the index sets *idx* [B][k], ordered as
    topk_ordered orders them (largest first, equal values by ascending index)."""
    asc = idx.sort(dim=-1).values
    vals = scores.gather(-1, asc)
    order = torch.sort(vals, dim=-1, descending=True, stable=True).indices
    return vals.gather(-1, order), asc.gather(-1, order)


def route_softmax_over(logits: torch.Tensor, idx: torch.Tensor):
    """route_softmax_topk's weights for a given expert set per row."""
    vals, idx = _over_set(torch.softmax(logits.float(), dim=-1), idx)
    return vals / vals.sum(dim=-1, keepdim=True), idx


def route_topk_softmax_over(logits: torch.Tensor, idx: torch.Tensor):
    """route_topk_softmax's weights for a given expert set per row."""
    vals, idx = _over_set(logits.float(), idx)
    return bf(torch.softmax(vals, dim=-1)), idx


def follow_near_ties(rlog: torch.Tensor, own: torch.Tensor, engine: torch.Tensor, k: int,
                     slack: float = 2.0):
    """Routing teacher-forced at near-ties, for whole-step parity tests.  Where a
    row's engine top-k set differs from the oracle's (*own*), the engine's set is
    taken if every expert it adds has an oracle logit at most *slack* bf16 ulps
    (of the k-th logit) below the k-th, and every expert it drops at most *slack*
    ulps above it: a near-tie that another f32 summation order settles the other
    way.  A difference past the slack is not followed and is reported.
    -> (index sets [B][k] i64, rows followed bool [B], rows past the slack bool [B],
    the largest distance of a swapped expert from the k-th logit in its ulps [B])"""
    B = rlog.shape[0]
    r = rlog.float()
    kth = r.sort(dim=-1, descending=True).values[:, k - 1]
    ulp = torch.exp2(torch.floor(torch.log2(kth.abs().clamp(min=2.0 ** -126))) - 7)
    out = own.clone().long()
    followed = torch.zeros(B, dtype=torch.bool)
    far = torch.zeros(B, dtype=torch.bool)
    dist = torch.zeros(B)
    for b in range(B):
        mine, theirs = set(own[b].tolist()), set(engine[b].tolist())
        if mine == theirs:
            continue
        swapped = [float(kth[b] - r[b, j]) for j in theirs - mine] + \
            [float(r[b, j] - kth[b]) for j in mine - theirs]
        dist[b] = max(swapped) / float(ulp[b])
        if dist[b] <= slack:
            followed[b] = True
            out[b] = torch.tensor(sorted(theirs), dtype=torch.long)
        else:
            far[b] = True
    return out, followed, far, dist


# ---------------------------------------------------------------------------
# Experts (a18, a22)
# ---------------------------------------------------------------------------
def moe_c4(x, weights, idx, w_gate, w_up, w_down, ws_gate, ws_up, ws_down, ws_scale):
    """Qwen3.5 routed + shared experts, torch_ref policy (torch_ref.py:451-530).

    x [B][H] (bf16 values), weights f32 [B][k], idx [B][k];
    w_gate/w_up [E][I][H], w_down [E][H][I] (out, in); shared ws_gate/ws_up
    [IS][H], ws_down [H][IS], ws_scale [1][H] (the (out, in) transposes of the
    reference's (in, out) shared weights).  -> f32 [B][H]."""
    B = x.shape[0]
    out = torch.zeros(B, w_down.shape[1])
    for b in range(B):
        xb = bf(x[b])
        routed = torch.zeros(w_down.shape[1])
        for s in range(idx.shape[1]):
            e = int(idx[b, s])
            g = bf(mm_rows(w_gate[e].float(), xb))
            u = bf(mm_rows(w_up[e].float(), xb))
            h = torch.nn.functional.silu(g) * u                  # f32
            d = bf(mm_rows(w_down[e].float(), bf(h)))            # _wm casts h to bf16
            routed = routed + d * weights[b, s].float()
        g = bf(mm_rows(ws_gate.float(), xb))
        u = bf(mm_rows(ws_up.float(), xb))
        dense = bf(mm_rows(ws_down.float(), bf(torch.nn.functional.silu(g) * u)))
        scale = torch.sigmoid(bf(mm_rows(ws_scale.float(), xb)))
        out[b] = routed + dense * scale
    return out


def moe_c5_dense(x, weights, idx, w_gate, w_up, w_down, w_shared_in, w_shared_out):
    """Granite routed experts + shared MLP at the HIR's rounding with the authored
    bf16 weights (model.py:406-471): w_gate/w_up [E][I][H], w_down [E][H][I],
    w_shared_in [2 IS][H], w_shared_out [H][IS].  -> bf16 values [B][H]."""
    B, H = x.shape
    out = torch.zeros(B, H)
    silu = torch.nn.functional.silu
    for b in range(B):
        xb = bf(x[b])
        weighted = []
        for s in range(idx.shape[1]):
            e = int(idx[b, s])
            g = bf(mm_rows(w_gate[e].float(), xb))
            u = bf(mm_rows(w_up[e].float(), xb))
            inner = bf(bf(silu(g)) * u)
            d = bf(mm_rows(w_down[e].float(), inner))
            weighted.append(bf(d * weights[b, s].float()))
        routed = bf(torch.stack(weighted).double().sum(dim=0).float())
        both = bf(mm_rows(w_shared_in.float(), xb))
        IS = w_shared_in.shape[0] // 2
        inner = bf(bf(silu(both[:IS])) * both[IS:])
        out[b] = bf(routed + bf(mm_rows(w_shared_out.float(), inner)))
    return out


def moe_c5(x, weights, idx, g_codes, g_scale, u_codes, u_scale, d_codes, d_scale,
           si_codes, si_scale, so_codes, so_scale):
    """Granite routed experts + shared MLP, HIR policy with fp8 weights
    (model.py:406-471).  x [B][H] (bf16 values), weights [B][k] (bf16 values);
    expert codes [E][I][H] / [E][H][I] with scales [E][I] / [E][H]; shared
    w_shared_in [2 IS][H] and w_shared_out [H][IS] as codes + per-row scales.
    -> bf16 values [B][H]."""
    B, H = x.shape
    out = torch.zeros(B, H)
    for b in range(B):
        xb = bf(x[b])
        weighted = []
        for s in range(idx.shape[1]):
            e = int(idx[b, s])
            g = bf(gemv_fp8(g_codes[e], g_scale[e], xb[None])[0])
            u = bf(gemv_fp8(u_codes[e], u_scale[e], xb[None])[0])
            inner = bf(bf(torch.nn.functional.silu(g)) * u)
            d = bf(gemv_fp8(d_codes[e], d_scale[e], inner[None])[0])
            weighted.append(bf(d * weights[b, s].float()))
        # tf.reduce(kind="sum") over the slots in bf16: one f32 sum, rounded once
        routed = bf(torch.stack(weighted).double().sum(dim=0).float())
        both = bf(gemv_fp8(si_codes, si_scale, xb[None])[0])
        IS = si_codes.shape[0] // 2
        inner = bf(bf(torch.nn.functional.silu(both[:IS])) * both[IS:])
        shared = bf(gemv_fp8(so_codes, so_scale, inner[None])[0])
        out[b] = bf(routed + shared)
    return out


# ---------------------------------------------------------------------------
# Gated DeltaNet decode step (a15), torch_ref policy
# ---------------------------------------------------------------------------
def conv_step_c4(conv_state, entry, conv_w):
    """``Qwen3_5LinearAttention.conv_step`` (tests/models/qwen3_5_35b_a3b/model.py:124-136;
    torch_ref f32): silu(sum(window * w)) over the window closing on `entry`.
    conv_state [B][C][K-1], entry [B][C] (f32) -> (mixed [B][C], the window [B][C][K])."""
    window = torch.cat((conv_state.float(), entry[:, :, None].float()), dim=2)
    return torch.nn.functional.silu((window * conv_w.float()[None]).sum(dim=-1)), window


def l2_normalise(x, eps=1e-6):
    """``l2_normalise`` (model.py:138-146): x * rsqrt(sum(x^2) + eps) over the last axis."""
    return x * torch.rsqrt(x.pow(2).sum(-1, keepdim=True) + eps)


def delta_step(state, q, k, v, g, beta, qscale):
    """``delta_step`` (model.py:148-172) with f64 sums: state [B][HV][DK][DV], q/k
    [B][HV][DK], v [B][HV][DV], g/beta [B][HV] -> (read f32 [B][HV][DV], updated f32)."""
    decayed = state.double() * torch.exp(g.double())[:, :, None, None]
    recalled = (decayed * k.double()[:, :, :, None]).sum(dim=2)
    delta = (v.double() - recalled) * beta.double()[:, :, None]
    updated = decayed + k.double()[:, :, :, None] * delta[:, :, None, :]
    read = (updated * (q.double() * qscale)[:, :, :, None]).sum(dim=2)
    return read.float(), updated.float()


def gdn_step(proj, conv_state, state, conv_w, a_log, dt_bias, gamma_gdn, *, hk, hv, dk, dv,
             l2_eps=1e-6, rms_eps=1e-6):
    """Everything of ``linear_attention`` between the in-projection and the
    out-projection (torch_ref.py:188-312; model.py:124-232), for a batch.

    proj  [B][2*KEY + VAL + 2*HV]: this token's projections, f32 of bf16 values,
          in the order [q | k | v] (the conv channels), z, b, a
    conv_state [B][CONV][KERNEL-1] f32, state [B][HV][DK][DV] f32,
    conv_w [CONV][KERNEL], a_log/dt_bias [HV], gamma_gdn [DV].
    -> (gated f32 [B][VAL] (before the out-projection's bf16 cast),
        new conv_state, new state)."""
    B = proj.shape[0]
    key, val = hk * dk, hv * dv
    conv = 2 * key + val
    entry = proj[:, :conv]
    z = proj[:, conv:conv + val]
    b_raw = proj[:, conv + val:conv + val + hv]
    a_raw = proj[:, conv + val + hv:conv + val + 2 * hv]
    mixed, window = conv_step_c4(conv_state, entry, conv_w)
    q = mixed[:, :key].reshape(B, hk, dk).repeat_interleave(hv // hk, dim=1)
    k = mixed[:, key:2 * key].reshape(B, hk, dk).repeat_interleave(hv // hk, dim=1)
    v = mixed[:, 2 * key:].reshape(B, hv, dv)
    q = l2_normalise(q, l2_eps)                                           # :206-216
    k = l2_normalise(k, l2_eps)
    beta = torch.sigmoid(b_raw)
    g = -torch.exp(a_log.float()) * torch.nn.functional.softplus(a_raw + dt_bias.float())
    read, updated = delta_step(state, q, k, v, g, beta, dk ** -0.5)      # :218-241
    # gated norm: _rms_norm(read, gamma_gdn) * silu(z), per value head
    normed = read * torch.rsqrt(read.pow(2).mean(-1, keepdim=True) + rms_eps) * gamma_gdn.float()
    gated = normed * torch.nn.functional.silu(z.reshape(B, hv, dv))
    new_conv = window[:, :, 1:].contiguous()
    return gated.reshape(B, val), new_conv, updated


# ---------------------------------------------------------------------------
# Mamba2 decode step (a19), HIR policy
# ---------------------------------------------------------------------------
def conv_step_c5(conv_state, entry, conv_w, conv_b):
    """``GraniteMamba.conv_step`` (examples/granite_4_0_h_small-cuda/model.py:154-168) at
    the HIR's rounding: bf16 window * kernel (each product rounded), the sum (f32,
    rounded once), + bias (rounded), silu (rounded).  conv_state [B][C][K-1], entry
    [B][C] (bf16 values) -> (mixed [B][C] bf16 values, the window [B][C][K])."""
    window = torch.cat((conv_state.float(), entry[:, :, None].float()), dim=2)
    weighted = bf(window * conv_w.float()[None])
    summed = bf(weighted.double().sum(dim=-1).float())
    return bf(torch.nn.functional.silu(bf(summed + conv_b.float()[None]))), window


def ssm_step(ssm_state, x, bvec, cvec, dt_raw, a_log, dt_bias, d_skip):
    """``GraniteMamba.ssm_step`` (model.py:170-221) at the HIR's rounding, f32 state.
    ssm_state [B][NH][PD][NS], x [B][NH][PD], bvec/cvec [B][NG][NS], dt_raw [B][NH]
    (bf16 values), a_log/dt_bias/d_skip [NH] -> (y bf16 values [B][NH][PD], updated)."""
    nh, ng = x.shape[1], bvec.shape[1]
    dt = bf(torch.nn.functional.softplus(bf(dt_raw + dt_bias.float()[None])))
    a = -torch.exp(a_log.float())
    decay = torch.exp(dt * a[None])                                          # f32
    hpg = nh // ng
    b_e = bvec.repeat_interleave(hpg, dim=1)[:, :, None, :]                  # [B][NH][1][NS]
    c_e = cvec.repeat_interleave(hpg, dim=1)[:, :, None, :]
    d_b = bf(dt[:, :, None, None] * b_e)
    d_bx = bf(d_b * x[:, :, :, None])
    updated = ssm_state.float() * decay[:, :, None, None] + d_bx
    read = (bf(updated).double() * c_e.double()).sum(dim=-1).float()
    y = bf(bf(read) + bf(x * d_skip.float()[None, :, None]))
    return y, updated


def gated_rmsnorm(y, gate, gamma, eps):
    """gated_out's RMSNormGated (model.py:223-237): the gate multiplies before the norm,
    f32, then one bf16 rounding.  y/gate [B][EXP] (bf16 values) -> bf16 values."""
    gated = y * torch.nn.functional.silu(gate)
    return bf(gated * torch.rsqrt(gated.pow(2).mean(-1, keepdim=True) + eps) * gamma.float())


def mamba_step(proj, conv_state, ssm_state, conv_w, conv_b, a_log, dt_bias, d_skip, gamma_ssm,
               *, nh, pd, ns, ng, eps=1e-5):
    """``mamba_mixer`` between ``in_projection`` and ``out_proj``
    (model.py:154-270): conv_step (:154-168), ssm_step (:170-221) and the
    RMSNormGated of gated_out (:223-238), for a batch.

    proj [B][EXP + CONV + NH] bf16 values: gate | x B C | dt_raw;
    conv_state [B][CONV][KRN-1] bf16 values; ssm_state [B][NH][PD][NS] f32;
    conv_w [CONV][KRN], conv_b [CONV], a_log/dt_bias/d_skip [NH], gamma_ssm [EXP].
    -> (normed bf16 values [B][EXP] (out_proj's input), new conv_state, new state)."""
    B = proj.shape[0]
    exp_ = nh * pd
    conv = exp_ + 2 * ng * ns
    gate = proj[:, :exp_]
    entry = proj[:, exp_:exp_ + conv]
    dt_raw = proj[:, exp_ + conv:exp_ + conv + nh]
    mixed, window = conv_step_c5(conv_state, entry, conv_w, conv_b)
    x = mixed[:, :exp_].reshape(B, nh, pd)
    bvec = mixed[:, exp_:exp_ + ng * ns].reshape(B, ng, ns)
    cvec = mixed[:, exp_ + ng * ns:].reshape(B, ng, ns)
    y, updated = ssm_step(ssm_state, x, bvec, cvec, dt_raw, a_log, dt_bias, d_skip)
    normed = gated_rmsnorm(y.reshape(B, exp_), gate, gamma_ssm, eps)
    new_conv = window[:, :, 1:].contiguous()
    return normed, new_conv, updated


# ---------------------------------------------------------------------------
# Full-attention layers of the hybrids, between the projections and o_proj
# ---------------------------------------------------------------------------
def _rotate_half(x):
    """HF ``rotate_half``: ``cat(-x[..., h:], x[..., :h])`` (torch_ref.py:157-162)."""
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def _rms_flat(x, w, eps):
    """``tf.rms_norm`` as torch_ref.py:145-154 spells it: flat in w, f32."""
    xf = x.float()
    return xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps) * w.float()


def partial_rope(x, cos, sin):
    """``partial_rope`` / ``partial_rope_kv`` (tests/models/qwen3_5_35b_a3b/model.py:
    235-262; torch_ref.py:165-181, f32): x [B][H][D], cos/sin [B][ROT] the rows at each
    sequence's position; the first ROT dims rotated half, the tail passed through."""
    rot = cos.shape[-1]
    r = x[..., :rot].float()
    c, s_ = cos.float()[:, None, :], sin.float()[:, None, :]
    return torch.cat((r * c + _rotate_half(r) * s_, x[..., rot:].float()), -1)


def qwen35_attend(qg, k, v, k_past, v_past, gamma_q, gamma_k, cos, sin, scale, eps=1e-6):
    """C4 (a16): ``full_attention`` of torch_ref.py:335-409 between the q/k/v
    projections and o_proj, for a batch of sequences each with its own past.

    qg [B][HQ][2D] f32 (bf16 values; query then output gate per head, the
    interleaving of :371-377), k/v [B][HKV][D] f32 (bf16 values); k_past[b],
    v_past[b] [C_b][HKV][D] (bf16 values, the cache before this token);
    gamma_q/gamma_k [D]; cos/sin [B][ROT] (the rows at each sequence's
    position); scale a float.  Per-head RMSNorm, rotate-half RoPE on the first
    ROT dims (_partial_rope :165-181), softmax over past + this token, output
    gate ``attn * sigmoid(gate)``.  Sums and the softmax in f64.
    -> (gated f32 [B][HQ*D] (o_proj's input before its bf16 cast),
        k_rope f32 [B][HKV][D] (the cache stores it rounded to bf16))."""
    B, HQ, D2 = qg.shape
    D = D2 // 2
    HKV = k.shape[1]
    G = HQ // HKV
    rot = cos.shape[-1]
    out = torch.zeros(B, HQ * D)
    k_rope = torch.zeros(B, HKV, D)

    def prope(x, b):
        r = x[:, :rot]
        return torch.cat((r * cos[b].float() + _rotate_half(r) * sin[b].float(), x[:, rot:]), -1)

    for b in range(B):
        q = qg[b, :, :D].float()
        gate = qg[b, :, D:].float()
        q_s = prope(_rms_flat(q, gamma_q, eps), b) * scale
        kr = prope(_rms_flat(k[b], gamma_k, eps), b)
        k_all = torch.cat((k_past[b].float(), kr[None]))
        v_all = torch.cat((v_past[b].float(), v[b][None].float()))
        kg = k_all.repeat_interleave(G, dim=1).double()           # [C+1][HQ][D]
        vg = v_all.repeat_interleave(G, dim=1).double()
        scores = (q_s.double()[None] * kg).sum(-1)                 # [C+1][HQ]
        probs = torch.softmax(scores, dim=0)
        attn = (probs[:, :, None] * vg).sum(0).float()             # [HQ][D]
        out[b] = (attn * torch.sigmoid(gate)).reshape(-1)
        k_rope[b] = kr
    return out, k_rope


def granite_attend(q, k_new, v_new, k_past, v_past, scale):
    """C5 (a20): ``GraniteAttention.attend`` (model.py:310-344) after
    ``cache_update`` at cur_pos (:362-364), for a batch: no position embedding,
    bf16 ops rounded as the HIR writes them, the softmax in f32 (here f64, then
    cast).  q [B][HQ][D], k_new/v_new [B][HKV][D], k_past[b]/v_past[b]
    [C_b][HKV][D], all bf16 values; scale the attention multiplier.  Masked
    positions contribute exp(-inf) = 0, so only positions 0..cur_pos are summed.
    -> attn bf16 values [B][HQ*D] (o_proj's input)."""
    B, HQ, D = q.shape
    HKV = k_new.shape[1]
    G = HQ // HKV
    out = torch.zeros(B, HQ * D)
    for b in range(B):
        k_all = torch.cat((k_past[b].float(), k_new[b][None].float()))
        v_all = torch.cat((v_past[b].float(), v_new[b][None].float()))
        kg = k_all.repeat_interleave(G, dim=1)                     # [C+1][HQ][D]
        vg = v_all.repeat_interleave(G, dim=1)
        scores = bf(bf(q[b].float()[None] * kg).double().sum(-1).float())
        scaled = scores * scale
        probs = bf(torch.softmax(scaled.double(), dim=0).float())
        out[b] = bf(bf(probs[:, :, None] * vg).double().sum(0).float()).reshape(-1)
    return out


# ---------------------------------------------------------------------------
# Whole decode steps of the C4 model (torch_ref policy)
# ---------------------------------------------------------------------------
def _rope_rows(theta, rot, rows):
    inv = 1.0 / theta ** (torch.arange(0, rot, 2, dtype=torch.float64) / rot)
    f = torch.arange(rows, dtype=torch.float64)[:, None] * inv[None]
    emb = torch.cat((f, f), dim=-1)
    return bf(emb.cos().float()), bf(emb.sin().float())


class Qwen35Oracle:
    """``Qwen3_5Decoder``'s decode step for a batch of sequences, composed from
    the torch twin's functions (torch_ref.py:243-312 linear_attention, :335-409
    full_attention, :417-530 routing / post_norm / experts, :533-575 residual_add,
    embed, final_rms_norm, lm_head): f32 residual stream, each matmul on the bf16
    cast of its input with one rounding of the sum.  Weights are CPU tensors in
    (out, in) row layouts under the names ``tilefoundry_amd.hybrid.qwen3_5``
    uses; `cfg` supplies the shape (layer i is full attention when
    ``cfg.is_full(i)``).  Each sequence carries its conv window, recurrent state
    and KV cache from step to step."""

    def __init__(self, cfg, weights: dict, rows: int, max_pos: int = 4096):
        self.cfg, self.w, self.B = cfg, weights, rows
        c = cfg
        self.conv = {i: torch.zeros(rows, c.conv_dim, c.conv_kernel - 1)
                     for i in range(c.layers) if not c.is_full(i)}
        self.state = {i: torch.zeros(rows, c.lin_value_heads, c.lin_key_dim, c.lin_value_dim)
                      for i in range(c.layers) if not c.is_full(i)}
        self.k_past = {i: [torch.zeros(0, c.kv_heads, c.head_dim)] * rows
                       for i in range(c.layers) if c.is_full(i)}
        self.v_past = {i: [torch.zeros(0, c.kv_heads, c.head_dim)] * rows
                       for i in range(c.layers) if c.is_full(i)}
        self.cos, self.sin = _rope_rows(c.rope_theta, c.rot_dim, max_pos)
        #: per step, per sequence: the smallest gap over layers between the k-th
        #: and (k+1)-th router logit, in bf16 ulps of the k-th (a gap of an ulp or
        #: two may pick another expert under any other summation order)
        self.route_gaps: list[torch.Tensor] = []
        #: per step, per sequence: the layers whose routing followed the engine's
        #: at a near-tie, and those whose engine set lay past the slack
        self.route_followed: list[torch.Tensor] = []
        self.route_far: list[torch.Tensor] = []
        #: per step, per sequence: the widest swap of the engine's routing, in
        #: ulps of the k-th logit, and the widest followed (follow_near_ties)
        self.route_dist: list[torch.Tensor] = []
        self.route_slack = 2.0

    def step(self, tokens, positions, routes=None) -> torch.Tensor:
        """One token per sequence at `positions` -> bf16-valued f32 logits [B][V].
        *routes*: the engine's top-k indices of this step [layers][B][k], followed
        at near-ties (follow_near_ties)."""
        c, B = self.cfg, self.B
        nfol = torch.zeros(B, dtype=torch.int64)
        nfar = torch.zeros(B, dtype=torch.int64)
        ndist = torch.zeros(B)
        hidden = self.w["embed"][torch.tensor(tokens)].float()
        pos = torch.tensor(positions)
        for i in range(c.layers):
            W = lambda n: self.w[f"layer{i}.{n}"]
            xn = bf(_rms_flat(hidden, W("gamma_in"), c.eps))
            proj = bf(mm_rows(W("w_in").float(), xn))
            if c.is_full(i):
                HQ, HKV, D = c.heads, c.kv_heads, c.head_dim
                qg = proj[:, :HQ * 2 * D].reshape(B, HQ, 2 * D)
                k = proj[:, HQ * 2 * D:HQ * 2 * D + HKV * D].reshape(B, HKV, D)
                v = proj[:, HQ * 2 * D + HKV * D:HQ * 2 * D + 2 * HKV * D].reshape(B, HKV, D)
                mixed, k_rope = qwen35_attend(qg, k, v, self.k_past[i], self.v_past[i],
                                              W("gamma_q"), W("gamma_k"), self.cos[pos],
                                              self.sin[pos], D ** -0.5, c.eps)
                self.k_past[i] = [torch.cat((self.k_past[i][b], bf(k_rope[b])[None]))
                                  for b in range(B)]
                self.v_past[i] = [torch.cat((self.v_past[i][b], v[b][None])) for b in range(B)]
            else:
                mixed, self.conv[i], self.state[i] = gdn_step(
                    proj, self.conv[i], self.state[i], W("conv_w"), W("a_log"), W("dt_bias"),
                    W("gamma_gdn"), hk=c.lin_key_heads, hv=c.lin_value_heads, dk=c.lin_key_dim,
                    dv=c.lin_value_dim, rms_eps=c.eps)
            hidden = hidden + bf(mm_rows(W("w_out").float(), bf(mixed)))
            xm = bf(_rms_flat(hidden, W("gamma_post"), c.eps))
            rlog = bf(mm_rows(W("w_router").float(), xm))
            srt = rlog.sort(dim=-1, descending=True).values
            kth = srt[:, c.top_k - 1].abs().clamp(min=2.0 ** -126)
            gap = (srt[:, c.top_k - 1] - srt[:, c.top_k]) / torch.exp2(torch.floor(torch.log2(kth)) - 7)
            gaps = gap if i == 0 else torch.minimum(gaps, gap)
            rw, ridx = route_softmax_topk(rlog, c.top_k)
            if routes is not None:
                use, fol, far, dist = follow_near_ties(rlog, ridx, routes[i], c.top_k,
                                                       self.route_slack)
                if fol.any():
                    rw, ridx = route_softmax_over(rlog, use)
                nfol += fol
                nfar += far
                ndist = torch.maximum(ndist, dist)
            IS = c.shared_inter
            hidden = hidden + moe_c4(xm, rw, ridx, W("w_gate"), W("w_up"), W("w_down"),
                                     W("w_shared_in")[:IS], W("w_shared_in")[IS:],
                                     W("w_shared_out"), W("w_shared_scale")[None])
        self.route_gaps.append(gaps)
        self.route_followed.append(nfol)
        self.route_far.append(nfar)
        self.route_dist.append(ndist)
        hn = bf(_rms_flat(hidden, self.w["gamma_final"], c.eps))
        return bf(mm_rows(self.w["head"].float(), hn))


# ---------------------------------------------------------------------------
# Whole decode steps of the C5 model (HIR policy, fp8 linear weights)
# ---------------------------------------------------------------------------
def rms_norm_tf(x, gamma, eps):
    """``tf.rms_norm`` as the evaluator values it (src/tilefoundry/ir/hir/nn/
    rms_norm.py:103-110): x and gamma in f32, ``x * rsqrt(mean(x^2) + eps) * gamma``
    in f32, rounded to bf16 once."""
    x32 = x.float()
    var = x32.pow(2).mean(dim=-1, keepdim=True)
    return bf(x32 * torch.rsqrt(var + eps) * gamma.float())


def _route_gap_ulps(rlog, k):
    srt = rlog.sort(dim=-1, descending=True).values
    kth = srt[:, k - 1].abs().clamp(min=2.0 ** -126)
    return (srt[:, k - 1] - srt[:, k]) / torch.exp2(torch.floor(torch.log2(kth)) - 7)


class GraniteOracle:
    """``Granite4_0_H_Small``'s decode step for a batch (examples/
    granite_4_0_h_small-cuda/model.py: embed :615-624, GraniteMamba :141-270,
    GraniteAttention :273-366, GraniteMoE :392-477, the layers' scaled residual
    :480-523, final norm and head :626-645, ``/ logits_scaling`` included) at the
    HIR's bf16 rounding, with every linear weight fp8 codes + f32 row scales
    (``gemv_fp8``) and the tied table bf16.  Weights under the names
    ``tilefoundry_amd.hybrid.granite`` uses, on the CPU."""

    def __init__(self, cfg, weights: dict, rows: int):
        self.cfg, self.w, self.B = cfg, weights, rows
        c = cfg
        self.conv = {i: torch.zeros(rows, c.conv_dim, c.conv_kernel - 1)
                     for i in range(c.layers) if not c.is_attention(i)}
        self.state = {i: torch.zeros(rows, c.mamba_heads, c.mamba_head_dim, c.d_state)
                      for i in range(c.layers) if not c.is_attention(i)}
        self.k_past = {i: [torch.zeros(0, c.kv_heads, c.head_dim)] * rows
                       for i in range(c.layers) if c.is_attention(i)}
        self.v_past = {i: [torch.zeros(0, c.kv_heads, c.head_dim)] * rows
                       for i in range(c.layers) if c.is_attention(i)}
        self.route_gaps: list[torch.Tensor] = []
        self.route_followed: list[torch.Tensor] = []
        self.route_far: list[torch.Tensor] = []
        #: per step, per sequence: the widest swap of the engine's routing, in
        #: ulps of the k-th logit, and the widest followed (follow_near_ties)
        self.route_dist: list[torch.Tensor] = []
        self.route_slack = 2.0

    def step(self, tokens, routes=None) -> torch.Tensor:
        """One token per sequence -> logits [B][V]; *routes* as Qwen35Oracle.step."""
        c, B = self.cfg, self.B
        nfol = torch.zeros(B, dtype=torch.int64)
        nfar = torch.zeros(B, dtype=torch.int64)
        ndist = torch.zeros(B)
        E, I, H = c.experts, c.moe_inter, c.hidden
        hidden = bf(self.w["embed"][torch.tensor(tokens)].float() * c.embedding_multiplier)
        gaps = None
        for i in range(c.layers):
            W = lambda n: self.w[f"layer{i}.{n}"]
            lin = lambda n, x: bf(gemv_fp8(W(n), W(n + "_scale"), x))
            xn = rms_norm_tf(hidden, W("gamma_in"), c.eps)
            if c.is_attention(i):
                HQ, HKV, D = c.heads, c.kv_heads, c.head_dim
                qkv = lin("w_in", xn)
                q = qkv[:, :HQ * D].reshape(B, HQ, D)
                k = qkv[:, HQ * D:(HQ + HKV) * D].reshape(B, HKV, D)
                v = qkv[:, (HQ + HKV) * D:(HQ + 2 * HKV) * D].reshape(B, HKV, D)
                att = granite_attend(q, k, v, self.k_past[i], self.v_past[i],
                                     c.attention_multiplier)
                self.k_past[i] = [torch.cat((self.k_past[i][b], k[b][None])) for b in range(B)]
                self.v_past[i] = [torch.cat((self.v_past[i][b], v[b][None])) for b in range(B)]
                mixed = lin("w_out", att)
            else:
                proj = lin("w_in", xn)
                normed, self.conv[i], self.state[i] = mamba_step(
                    proj, self.conv[i], self.state[i], W("conv_w"), W("conv_b"), W("a_log"),
                    W("dt_bias"), W("d_skip"), W("gamma_ssm"), nh=c.mamba_heads,
                    pd=c.mamba_head_dim, ns=c.d_state, ng=1, eps=c.eps)
                mixed = lin("w_out", normed)
            hidden = bf(hidden + bf(mixed * c.residual_multiplier))
            xm = rms_norm_tf(hidden, W("gamma_post"), c.eps)
            rlog = lin("w_router", xm)
            gap = _route_gap_ulps(rlog, c.top_k)
            gaps = gap if gaps is None else torch.minimum(gaps, gap)
            rw, ridx = route_topk_softmax(rlog, c.top_k)
            if routes is not None:
                use, fol, far, dist = follow_near_ties(rlog, ridx, routes[i], c.top_k,
                                                       self.route_slack)
                if fol.any():
                    rw, ridx = route_topk_softmax_over(rlog, use)
                nfol += fol
                nfar += far
                ndist = torch.maximum(ndist, dist)
            moe = moe_c5(xm, rw, ridx, W("w_gate").view(E, I, H), W("s_gate").view(E, I),
                         W("w_up").view(E, I, H), W("s_up").view(E, I),
                         W("w_down").view(E, H, I), W("s_down").view(E, H),
                         W("w_shared_in"), W("w_shared_in_scale"), W("w_shared_out"),
                         W("w_shared_out_scale"))
            hidden = bf(hidden + bf(moe * c.residual_multiplier))
        self.route_gaps.append(gaps)
        self.route_followed.append(nfol)
        self.route_far.append(nfar)
        self.route_dist.append(ndist)
        hn = rms_norm_tf(hidden, self.w["gamma_final"], c.eps)
        return bf(bf(mm_rows(self.w["embed"].float(), hn)) / c.logits_scaling)
