// The hybrid mixers' authored sub-functions as kernels of their own.
//
// The decode engines run each mixer as one fused launch (tfd_gdn_step,
// tfd_mamba_step in hybrid.hip).  The reference's runtime twins, though, keep
// every authored @func callable by itself (src/tilefoundry/runtime/
// decorator.py:182-192 requires the twin's function set to equal the authored
// one), so a caller can drive conv_step, l2_normalise, delta_step,
// partial_rope, ssm_step and gated_out one at a time.  These kernels are those
// functions, with the arithmetic of the fused launches (which follow the
// reference: C4 at the torch twin's f32 policy, examples/qwen3_5_35b_a3b-
// tilelang/kernels/torch_ref.py:22-40; C5 at the Granite HIR's bf16 rounding,
// examples/granite_4_0_h_small-cuda/model.py).  They are small, one-token
// kernels: a block per row (and head), no work buffers.
#include "hybrid_common.h"
#include "host_common.h"
#include "tf_hybrid.h"

using namespace tfd;
using namespace tfd_host;
using namespace tfd_hybrid;

namespace {

// ---------------------------------------------------------------------------
// conv_step (C4: tests/models/qwen3_5_35b_a3b/model.py:124-136, torch_ref f32;
// C5: examples/granite_4_0_h_small-cuda/model.py:154-168, bf16 ops): the window
// closes on this token's entry, one product per tap, summed, (+ bias), SiLU.
// ---------------------------------------------------------------------------
template <bool kBf16>
__global__ __launch_bounds__(kBlock) void k_conv_step(TfdConvStepArgs a) {
  constexpr int kKW = 4;
  const int b = blockIdx.y, c = blockIdx.x * kBlock + threadIdx.x;
  if (c >= a.channels) return;
  const bf16* w = (const bf16*)a.conv_w + (int64_t)c * kKW;
  float win[kKW];
  if (kBf16) {
    const bf16* s = (const bf16*)a.window + ((int64_t)b * a.channels + c) * (kKW - 1);
#pragma unroll
    for (int t = 0; t < kKW - 1; ++t) win[t] = bf2f(s[t]);
    win[kKW - 1] = bf2f(((const bf16*)a.entry)[(int64_t)b * a.lde + c]);
    float sum = 0.f;
#pragma unroll
    for (int t = 0; t < kKW; ++t) sum += rbf(win[t] * bf2f(w[t]));     // bf16 window * kernel
    const float pre = a.conv_b ? rbf(rbf(sum) + bf2f(((const bf16*)a.conv_b)[c])) : rbf(sum);
    ((bf16*)a.out)[(int64_t)b * a.ldo + c] = f2bf(silu_f(pre));
  } else {
    const float* s = (const float*)a.window + ((int64_t)b * a.channels + c) * (kKW - 1);
#pragma unroll
    for (int t = 0; t < kKW - 1; ++t) win[t] = s[t];
    win[kKW - 1] = ((const float*)a.entry)[(int64_t)b * a.lde + c];
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < kKW; ++t) acc += win[t] * bf2f(w[t]);
    if (a.conv_b) acc += bf2f(((const bf16*)a.conv_b)[c]);
    ((float*)a.out)[(int64_t)b * a.ldo + c] = silu_f(acc);
  }
}

// ---------------------------------------------------------------------------
// l2_normalise (model.py:138-146): x * rsqrt(sum(x^2) + eps) per vector, f32.
// One wave per vector of dim <= 256.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void k_l2norm(const float* __restrict__ x, float* __restrict__ out,
                                                   int nvec, int dim, float eps) {
  const int v = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (v >= nvec) return;
  const float* xv = x + (int64_t)v * dim;
  float e[4];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + kWave * i;
    e[i] = d < dim ? xv[d] : 0.f;
    ss += e[i] * e[i];
  }
  const float r = rsqrtf(wave_sum(ss) + eps);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + kWave * i;
    if (d < dim) out[(int64_t)v * dim + d] = e[i] * r;
  }
}

// ---------------------------------------------------------------------------
// delta_step (model.py:148-172): one token of the gated delta rule on an f32
// state, as the fused GDN launch computes it: thread (dv, half) owns key rows
// [half * DK/2, +DK/2) of column dv.
// ---------------------------------------------------------------------------
template <int kD>
__global__ __launch_bounds__(2 * kD) void k_delta_step(TfdDeltaStepArgs a) {
  const int hv = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int dv = tid % kD, half = tid / kD;
  constexpr int kRows = kD / 2;
  const int64_t head = (int64_t)b * a.heads + hv;
  __shared__ float q_s[kD], k_s[kD], red[2][kD];
  const float* si = a.state_in + (head * kD + half * kRows) * kD + dv;
  float* so = a.state_out + (head * kD + half * kRows) * kD + dv;
  float s[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) s[r] = si[(int64_t)r * kD];
  if (tid < kD) {
    q_s[tid] = a.q[head * kD + tid] * a.qscale;
    k_s[tid] = a.k[head * kD + tid];
  }
  __syncthreads();
  const float decay = expf(a.g[head]), beta = a.beta[head];
  float rec = 0.f;
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    s[r] *= decay;
    rec += s[r] * k_s[half * kRows + r];
  }
  red[half][dv] = rec;
  __syncthreads();
  const float delta = (a.v[head * kD + dv] - (red[0][dv] + red[1][dv])) * beta;
  float rd = 0.f;
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const float u = s[r] + k_s[half * kRows + r] * delta;
    so[(int64_t)r * kD] = u;
    rd += u * q_s[half * kRows + r];
  }
  __syncthreads();
  red[half][dv] = rd;
  __syncthreads();
  if (tid < kD) a.read[head * kD + tid] = red[0][tid] + red[1][tid];
}

// ---------------------------------------------------------------------------
// partial_rope / partial_rope_kv (model.py:235-262, torch_ref f32): the first
// rot dims of each head rotated half against the cos/sin rows at pos (bf16
// tables), the tail passed through.  Thread per (row, head, dim).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void k_partial_rope(TfdPartialRopeArgs a) {
  const int b = blockIdx.y;
  const int i = blockIdx.x * kBlock + threadIdx.x;
  const int n = a.heads * a.head_dim;
  if (i >= n) return;
  const int d = i % a.head_dim, h0 = i - d;
  const float* xr = a.x + (int64_t)b * a.ldx;
  float y = xr[i];
  if (d < a.rot) {
    const int half = a.rot / 2;
    const int p = a.pos[b];
    const int64_t row = (int64_t)((p >= 0 && p < a.rope_rows) ? p : 0) * a.rot;
    const float c = bf2f(((const bf16*)a.cos_table)[row + d]);
    const float sn = bf2f(((const bf16*)a.sin_table)[row + d]);
    const float rot = d < half ? -xr[h0 + d + half] : xr[h0 + d - half];
    y = y * c + rot * sn;
  }
  a.out[(int64_t)b * a.ldo + i] = y;
}

// ---------------------------------------------------------------------------
// ssm_step (examples/granite_4_0_h_small-cuda/model.py:170-221): the
// selective-state update of one token with bf16 ops rounded as the HIR writes
// them and an f32 state; one block per (head, row), a state row's 128 columns
// as 32 lanes x 4.  ngroups 1, head_dim 64, d_state 128.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void k_ssm_step(TfdSsmStepArgs a) {
  constexpr int kPD = 64, kNS = 128;
  constexpr int kLpr = kNS / 4, kRpp = kBlock / kLpr, kPass = kPD / kRpp;
  const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int q = tid % kLpr, r0 = tid / kLpr;
  const int64_t head = (int64_t)b * a.heads + h;
  const float4* si = reinterpret_cast<const float4*>(a.state_in + head * kPD * kNS) + q;
  float4* so = reinterpret_cast<float4*>(a.state_out + head * kPD * kNS) + q;
  __shared__ float x_s[kPD];
  __shared__ float dtv[2];
  float4 sv[kPass];
#pragma unroll
  for (int i = 0; i < kPass; ++i) sv[i] = si[(int64_t)(r0 + kRpp * i) * kLpr];
  const bf16* xr = (const bf16*)a.x + (int64_t)b * a.ldx + h * kPD;
  if (tid < kPD) x_s[tid] = bf2f(xr[tid]);
  if (tid == 0) {
    const float raw = bf2f(((const bf16*)a.dt_raw)[(int64_t)b * a.lddt + h]);
    const float dt = rbf(softplus_f(rbf(raw + bf2f(((const bf16*)a.dt_bias)[h]))));
    dtv[0] = dt;
    dtv[1] = expf(dt * -expf(bf2f(((const bf16*)a.a_log)[h])));
  }
  __syncthreads();
  const float dt = dtv[0], decay = dtv[1];
  const bf16* bv = (const bf16*)a.b_vec + (int64_t)b * a.ldb;
  const bf16* cv = (const bf16*)a.c_vec + (int64_t)b * a.ldc;
  float dtb[4], cq[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    dtb[e] = rbf(dt * bf2f(bv[4 * q + e]));
    cq[e] = bf2f(cv[4 * q + e]);
  }
  const float dsk = bf2f(((const bf16*)a.d_skip)[h]);
#pragma unroll
  for (int i = 0; i < kPass; ++i) {
    const int p = r0 + kRpp * i;
    const float xp = x_s[p];
    float u[4] = {sv[i].x, sv[i].y, sv[i].z, sv[i].w};
    float rd = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      u[e] = u[e] * decay + rbf(dtb[e] * xp);
      rd += rbf(u[e]) * cq[e];
    }
    so[(int64_t)p * kLpr] = float4{u[0], u[1], u[2], u[3]};
    rd = group_sum<kLpr>(rd);
    if (q == 0)
      ((bf16*)a.y)[(int64_t)b * a.ldy + h * kPD + p] = f2bf(rbf(rd) + rbf(xp * dsk));
  }
}

// ---------------------------------------------------------------------------
// gated_out's RMSNormGated (model.py:223-237): gated = f32(y) * silu(f32(gate)),
// then x * rsqrt(mean(x^2) + eps) * gamma in f32, rounded to bf16 once.  One
// block per row of n <= 8192 values.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void k_gated_rmsnorm(TfdGatedNormArgs a) {
  constexpr int kMax = 32;
  const int b = blockIdx.x, tid = threadIdx.x;
  const bf16* y = (const bf16*)a.y + (int64_t)b * a.ldy;
  const bf16* g = (const bf16*)a.gate + (int64_t)b * a.ldg;
  __shared__ float red[kWavesPerBlock];
  float v[kMax];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kMax; ++i) {
    const int c = tid + kBlock * i;
    v[i] = c < a.n ? bf2f(y[c]) * silu_f(bf2f(g[c])) : 0.f;
    ss += v[i] * v[i];
  }
  ss = wave_sum(ss);
  if ((tid & (kWave - 1)) == 0) red[tid / kWave] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < kWavesPerBlock; ++w) tot += red[w];
  const float r = rsqrtf(tot / (float)a.n + a.eps);
  bf16* o = (bf16*)a.out + (int64_t)b * a.ldo;
#pragma unroll
  for (int i = 0; i < kMax; ++i) {
    const int c = tid + kBlock * i;
    if (c < a.n) o[c] = f2bf(v[i] * r * bf2f(((const bf16*)a.gamma)[c]));
  }
}

}  // namespace

extern "C" {

int tfd_conv_step_rows(const TfdConvStepArgs* args, void* stream) {
  if (!args) return fail(kBadArg, "conv_step: null args");
  const TfdConvStepArgs& a = *args;
  if (!a.window || !a.entry || !a.conv_w || !a.out)
    return fail(kBadArg, "conv_step: null pointer");
  if (a.rows <= 0 || a.channels <= 0 || a.kernel != 4 || a.lde < a.channels ||
      a.ldo < a.channels)
    return fail(kBadShape, "conv_step: rows %d, channels %d, kernel %d (4 only), lde %d, ldo %d",
                a.rows, a.channels, a.kernel, a.lde, a.ldo);
  const dim3 g((a.channels + kBlock - 1) / kBlock, a.rows);
  if (a.policy == TFD_POLICY_BF16)
    hipLaunchKernelGGL(k_conv_step<true>, g, dim3(kBlock), 0, (hipStream_t)stream, a);
  else if (a.policy == TFD_POLICY_F32)
    hipLaunchKernelGGL(k_conv_step<false>, g, dim3(kBlock), 0, (hipStream_t)stream, a);
  else
    return fail(kBadArg, "conv_step: policy %d", a.policy);
  return launched("conv_step");
}

int tfd_l2norm_f32(const float* x, float* out, int nvec, int dim, float eps, void* stream) {
  if (!x || !out) return fail(kBadArg, "l2norm: null pointer");
  if (nvec <= 0 || dim <= 0 || dim > 4 * kWave)
    return fail(kBadShape, "l2norm: %d vectors of %d (dim <= 256)", nvec, dim);
  hipLaunchKernelGGL(k_l2norm, dim3((nvec + kWavesPerBlock - 1) / kWavesPerBlock),
                     dim3(kBlock), 0, (hipStream_t)stream, x, out, nvec, dim, eps);
  return launched("l2norm");
}

int tfd_delta_step_f32(const TfdDeltaStepArgs* args, void* stream) {
  if (!args) return fail(kBadArg, "delta_step: null args");
  const TfdDeltaStepArgs& a = *args;
  if (!a.state_in || !a.state_out || !a.q || !a.k || !a.v || !a.g || !a.beta || !a.read)
    return fail(kBadArg, "delta_step: null pointer");
  if (a.rows <= 0 || a.heads <= 0 || a.head_k_dim != 128 || a.head_v_dim != 128)
    return fail(kBadShape, "delta_step: rows %d, heads %d, dims %d x %d (128 x 128 only)",
                a.rows, a.heads, a.head_k_dim, a.head_v_dim);
  hipLaunchKernelGGL(k_delta_step<128>, dim3(a.heads, a.rows), dim3(256), 0,
                     (hipStream_t)stream, a);
  return launched("delta_step");
}

int tfd_partial_rope_f32(const TfdPartialRopeArgs* args, void* stream) {
  if (!args) return fail(kBadArg, "partial_rope: null args");
  const TfdPartialRopeArgs& a = *args;
  if (!a.x || !a.out || !a.pos || !a.cos_table || !a.sin_table)
    return fail(kBadArg, "partial_rope: null pointer");
  const int n = a.heads * a.head_dim;
  if (a.rows <= 0 || n <= 0 || a.rot <= 0 || a.rot > a.head_dim || a.rot % 2 || a.ldx < n ||
      a.ldo < n || a.rope_rows <= 0)
    return fail(kBadShape, "partial_rope: rows %d, %d heads of %d, rot %d", a.rows, a.heads,
                a.head_dim, a.rot);
  hipLaunchKernelGGL(k_partial_rope, dim3((n + kBlock - 1) / kBlock, a.rows), dim3(kBlock), 0,
                     (hipStream_t)stream, a);
  return launched("partial_rope");
}

int tfd_ssm_step_bf16(const TfdSsmStepArgs* args, void* stream) {
  if (!args) return fail(kBadArg, "ssm_step: null args");
  const TfdSsmStepArgs& a = *args;
  if (!a.state_in || !a.state_out || !a.x || !a.b_vec || !a.c_vec || !a.dt_raw || !a.a_log ||
      !a.dt_bias || !a.d_skip || !a.y)
    return fail(kBadArg, "ssm_step: null pointer");
  if (a.rows <= 0 || a.heads <= 0 || a.head_dim != 64 || a.state_dim != 128 ||
      a.ldx < a.heads * 64 || a.ldy < a.heads * 64 || a.ldb < 128 || a.ldc < 128 ||
      a.lddt < a.heads)
    return fail(kBadShape, "ssm_step: rows %d, %d heads of %d, state %d (64 x 128 only)",
                a.rows, a.heads, a.head_dim, a.state_dim);
  hipLaunchKernelGGL(k_ssm_step, dim3(a.heads, a.rows), dim3(kBlock), 0, (hipStream_t)stream, a);
  return launched("ssm_step");
}

int tfd_gated_rmsnorm_bf16(const TfdGatedNormArgs* args, void* stream) {
  if (!args) return fail(kBadArg, "gated_rmsnorm: null args");
  const TfdGatedNormArgs& a = *args;
  if (!a.y || !a.gate || !a.gamma || !a.out) return fail(kBadArg, "gated_rmsnorm: null pointer");
  if (a.rows <= 0 || a.n <= 0 || a.n > 32 * kBlock || a.ldy < a.n || a.ldg < a.n || a.ldo < a.n)
    return fail(kBadShape, "gated_rmsnorm: %d rows of %d (n <= 8192)", a.rows, a.n);
  hipLaunchKernelGGL(k_gated_rmsnorm, dim3(a.rows), dim3(kBlock), 0, (hipStream_t)stream, a);
  return launched("gated_rmsnorm");
}

}  // extern "C"
