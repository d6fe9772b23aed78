// Small-batch (1..4 sequences) decode kernels for the Qwen3.5 hybrid (workload
// C4 at batch 1), where a step is latency-bound: every launch is short, so the
// step is cut to fewer, wider launches and no projection pads its rows up to an
// MFMA tile.
//
// A gated-DeltaNet layer is six launches instead of ten (the reference's
// tilelang runtime also runs the mixer as three kernels, examples/
// qwen3_5_35b_a3b-tilelang/kernels/gdn.py:1-60):
//   in-proj   row GEMV with the input RMSNorm as its prologue (every block
//             normalises the f32 residual row itself: 8 KB from the L2)
//   delta     the conv + l2norm + delta rule split over value columns, 32 per
//             block: 128 blocks at batch 1 instead of 32 (a value column needs
//             only its own state column, gdn.py:47-60)
//   out-proj  row GEMV whose prologue is the gated RMS norm of the read-out
//             (per head, the same sums as tfd_gdn_step), adding into the f32
//             residual stream
//   router    row GEMV with the post norm as its prologue; block 0 also writes
//             the normalised rows the experts read
//   gate/up   every block routes its sequence itself (softmax, top-k, the
//             reference's moe.py:271-302 select) from the 256 logits, then
//             streams its expert's rows; the shared expert needs no routing and
//             starts at once
//   down+mix  per output row, the down rows of all picked experts and the
//             shared one, mixed in slot order and added into the stream
// The row GEMV keeps weights row-major ([N][K], a row one contiguous dot
// product); a wave owns kG rows, its lanes 16-byte chunks c = lane + 64 i.
//
// Arithmetic is the C4 policy (torch_ref.py:22-40): f32 activations, bf16
// matmul inputs, one bf16 rounding of each f32 sum.  The norms, the delta
// rule's read-out and the experts are computed exactly as the batched kernels
// compute them (same lanes, same summation order), so they agree bit for bit;
// only the GEMV's dot products are summed in another order than the MFMA
// GEMM's.
#include "hybrid_common.h"
#include "host_common.h"
#include "tf_decode.h"
#include "tf_hybrid.h"

#include <algorithm>

using namespace tfd;
using namespace tfd_host;
using namespace tfd_hybrid;

namespace {

constexpr int kSmallRows = 4;

// ---------------------------------------------------------------------------
// Row GEMV: out[r][n] (op)= bf16(sum_k W[n][k] x[r][k]) for r < rows <= 4.
// The input rows are staged into LDS as bf16 by a prologue of kind kX; the
// prologue's loads are issued before the first group's weight loads so that
// waiting for them does not wait for the weights (loads retire in order).
// ---------------------------------------------------------------------------
template <int kC>
struct XStage {
  static constexpr int kK = kC * 512;                 // values per row
  uint32_t w[kSmallRows][kK / 2];                     // bf16 pairs
};

// A group's weights, and with the residual epilogue the current values of its
// outputs (lane g < kG holds output g of every row), requested together so the
// read-modify-write at the end needs no round trip of its own.
template <int kEpi, int kC, int kG>
__device__ __forceinline__ void rg_issue(const TfdRowGemvArgs& a, const bf16* __restrict__ W,
                                         int grp, int lane, u32x4 (&w)[kG][kC],
                                         float (&res)[kSmallRows]) {
  constexpr int K = kC * 512;
#pragma unroll
  for (int g = 0; g < kG; ++g) {
    int n = grp * kG + g;
    n = n < a.N ? n : a.N - 1;
#pragma unroll
    for (int i = 0; i < kC; ++i) w[g][i] = load16_stream(W + (int64_t)n * K + (lane + kWave * i) * 8);
  }
  if constexpr (kEpi == TFD_EPI_RESID_F32) {
    int n = grp * kG + (lane < kG ? lane : 0);
    n = n < a.N ? n : a.N - 1;
#pragma unroll
    for (int r = 0; r < kSmallRows; ++r)
      res[r] = a.out[(int64_t)(r < a.rows ? r : 0) * a.ldo + n];
  }
}

template <int kEpi, int kC, int kG>
__device__ __forceinline__ void rg_finish(const TfdRowGemvArgs& a, const XStage<kC>& xs, int grp,
                                          int lane, const u32x4 (&w)[kG][kC],
                                          const float (&res)[kSmallRows]) {
#pragma unroll
  for (int r = 0; r < kSmallRows; ++r) {
    if (r >= a.rows) break;
    float acc[kG];
#pragma unroll
    for (int g = 0; g < kG; ++g) acc[g] = 0.f;
#pragma unroll
    for (int i = 0; i < kC; ++i) {
      const u32x4 x = *reinterpret_cast<const u32x4*>(&xs.w[r][(lane + kWave * i) * 4]);
#pragma unroll
      for (int g = 0; g < kG; ++g) acc[g] = dot8(w[g][i], x, acc[g]);
    }
#pragma unroll
    for (int g = 0; g < kG; ++g) {
      const float y = rbf(wave_sum(acc[g]));
      const int n = grp * kG + g;
      if (lane == g && n < a.N)
        a.out[(int64_t)r * a.ldo + n] = kEpi == TFD_EPI_RESID_F32 ? res[r] + y : y;
    }
  }
}

template <int kX, int kEpi, int kC, int kG>
__global__ __launch_bounds__(kBlock) void k_rowgemv(TfdRowGemvArgs a) {
  constexpr int K = kC * 512;
  __shared__ XStage<kC> xs;
  __shared__ float red[kSmallRows][kWavesPerBlock];
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int R = a.rows;
  const bf16* W = (const bf16*)a.w;
  const int ngroups = (a.N + kG - 1) / kG;
  const int tw = (int)gridDim.x * kWavesPerBlock;
  int grp = (int)blockIdx.x * kWavesPerBlock + wave;
  const bool write_rows = a.x_rows && blockIdx.x == 0;

  // ---- prologue loads
  constexpr int kN4 = K / 1024;                 // NORM: float4 per thread and row
  constexpr int kHw = K / 512;                  // GATED: heads per wave (128 values each)
  constexpr int kCh = K / 2048;                 // OPERAND / ROWS: 16-byte chunks per thread and row
  float4 nv[kSmallRows][kX == TFD_ROWX_NORM_F32 ? kN4 : 1];
  float gv[kSmallRows][kX == TFD_ROWX_GATED_F32 ? kHw : 1][4];
  u32x4 cv[kSmallRows][(kX == TFD_ROWX_OPERAND || kX == TFD_ROWX_ROWS) ? kCh : 1];
#pragma unroll
  for (int r = 0; r < kSmallRows; ++r) {
    const int rr = r < R ? r : 0;
    if constexpr (kX == TFD_ROWX_NORM_F32) {
      const float4* xr = reinterpret_cast<const float4*>((const float*)a.x + (int64_t)rr * a.ldx);
#pragma unroll
      for (int i = 0; i < kN4; ++i) nv[r][i] = xr[tid + kBlock * i];
    } else if constexpr (kX == TFD_ROWX_GATED_F32) {
      const float* xr = (const float*)a.x + (int64_t)rr * a.ldx;
      const float* zr = a.gate + (int64_t)rr * a.ldg;
#pragma unroll
      for (int j = 0; j < kHw; ++j) {
        const int c = (wave + kWavesPerBlock * j) * 128 + lane;
        gv[r][j][0] = xr[c];
        gv[r][j][1] = xr[c + 64];
        gv[r][j][2] = zr[c];
        gv[r][j][3] = zr[c + 64];
      }
    } else {
#pragma unroll
      for (int j = 0; j < kCh; ++j) {
        const int c = tid + kBlock * j;
        const bf16* src = kX == TFD_ROWX_OPERAND
                              ? (const bf16*)a.x + xp_off_h(rr, 8 * c)
                              : (const bf16*)a.x + (int64_t)rr * a.ldx + 8 * c;
        cv[r][j] = load16(src);
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  u32x4 wa[kG][kC], wb[kG][kC];
  float ra[kSmallRows], rb[kSmallRows];
  rg_issue<kEpi, kC, kG>(a, W, grp < ngroups ? grp : ngroups - 1, lane, wa, ra);
  __builtin_amdgcn_sched_barrier(0);

  // ---- prologue compute: the bf16 input rows into LDS
  if constexpr (kX == TFD_ROWX_NORM_F32) {
    // tfd_rmsnorm_f32_rows' arithmetic: per-thread squares in this order, the
    // wave sums, then the four waves' sums in wave order
#pragma unroll
    for (int r = 0; r < kSmallRows; ++r) {
      if (r >= R) break;
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < kN4; ++i) {
        const float4 v = nv[r][i];
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
      }
      ss = wave_sum(ss);
      if (lane == 0) red[r][wave] = ss;
    }
    __syncthreads();
    const bf16* gamma = (const bf16*)a.gamma;
#pragma unroll
    for (int r = 0; r < kSmallRows; ++r) {
      if (r >= R) break;
      float tot = 0.f;
#pragma unroll
      for (int w = 0; w < kWavesPerBlock; ++w) tot += red[r][w];
      const float rs = rsqrtf(tot / (float)K + a.eps);
#pragma unroll
      for (int i = 0; i < kN4; ++i) {
        const int q = tid + kBlock * i, c = 4 * q;
        const float4 v = nv[r][i];
        const uint2 g = *reinterpret_cast<const uint2*>(gamma + c);
        const uint2 o = {pack2(v.x * rs * bf_lo(g.x), v.y * rs * bf_hi(g.x)),
                         pack2(v.z * rs * bf_lo(g.y), v.w * rs * bf_hi(g.y))};
        *reinterpret_cast<uint2*>(&xs.w[r][2 * q]) = o;
        if (write_rows) *reinterpret_cast<uint2*>((bf16*)a.x_rows + (int64_t)r * a.ldxr + c) = o;
      }
    }
  } else if constexpr (kX == TFD_ROWX_GATED_F32) {
    // tfd_gdn_step's gated norm per head: the two 64-value halves' wave sums,
    // in order, over 128; then x * rsqrt(ms + eps) * gamma * silu(z)
    const bf16* gamma = (const bf16*)a.gamma;
    const float g0 = bf2f(gamma[lane]), g1 = bf2f(gamma[lane + 64]);
    bf16* xsh = reinterpret_cast<bf16*>(&xs.w[0][0]);
#pragma unroll
    for (int r = 0; r < kSmallRows; ++r) {
      if (r >= R) break;
#pragma unroll
      for (int j = 0; j < kHw; ++j) {
        const float s0 = wave_sum(gv[r][j][0] * gv[r][j][0]);
        const float s1 = wave_sum(gv[r][j][1] * gv[r][j][1]);
        float ms = 0.f;
        ms += s0;
        ms += s1;
        ms /= 128.f;
        const float rs = rsqrtf(ms + a.eps);
        const int c = (wave + kWavesPerBlock * j) * 128 + lane;
        const bf16 y0 = f2bf(gv[r][j][0] * rs * g0 * silu_f(gv[r][j][2]));
        const bf16 y1 = f2bf(gv[r][j][1] * rs * g1 * silu_f(gv[r][j][3]));
        xsh[(int64_t)r * K + c] = y0;
        xsh[(int64_t)r * K + c + 64] = y1;
        if (write_rows) {
          ((bf16*)a.x_rows)[(int64_t)r * a.ldxr + c] = y0;
          ((bf16*)a.x_rows)[(int64_t)r * a.ldxr + c + 64] = y1;
        }
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < kSmallRows; ++r) {
      if (r >= R) break;
#pragma unroll
      for (int j = 0; j < kCh; ++j) {
        const int c = tid + kBlock * j;
        *reinterpret_cast<u32x4*>(&xs.w[r][4 * c]) = cv[r][j];
        if (write_rows)
          *reinterpret_cast<u32x4*>((bf16*)a.x_rows + (int64_t)r * a.ldxr + 8 * c) = cv[r][j];
      }
    }
  }
  __syncthreads();

  // ---- groups of kG rows, two register sets in turn: the next group's
  // weights are requested before this group's products
  if (grp < ngroups) for (;;) {
    const int g1 = grp + tw;
    if (g1 < ngroups) rg_issue<kEpi, kC, kG>(a, W, g1, lane, wb, rb);
    rg_finish<kEpi, kC, kG>(a, xs, grp, lane, wa, ra);
    grp = g1;
    if (grp >= ngroups) break;
    const int g2 = grp + tw;
    if (g2 < ngroups) rg_issue<kEpi, kC, kG>(a, W, g2, lane, wa, ra);
    rg_finish<kEpi, kC, kG>(a, xs, grp, lane, wb, rb);
    grp = g2;
    if (grp >= ngroups) break;
  }
}

// ---------------------------------------------------------------------------
// Gated DeltaNet over value columns: block (value head, column group, row),
// 2 kCols threads.  Thread (column, half) holds its column's state over half
// of the key rows, as in tfd_gdn_step, and every per-column value (recalled,
// delta, the updated column, the read-out) is computed in that kernel's order,
// so the read-out is bit-identical to it.  The conv, l2 norms, beta and g of
// the head are recomputed by each of its column groups (a few hundred values);
// the q/k conv windows are advanced by the first value head of the key head's
// first group, the v windows by the group that owns them.  The read-out goes
// out in f32, un-normalised: the gated norm needs all of a head's columns and
// is the out-projection's prologue.
// ---------------------------------------------------------------------------
template <int kCols>
__global__ __launch_bounds__(2 * kCols) void k_gdn_cols(TfdGdnArgs t, float* __restrict__ read,
                                                         int ldr) {
  constexpr int kD = 128, kKW = 4, kRows = kD / 2, kT = 2 * kCols;
  static_assert(kT == kWave, "one wave per block");
  const int hv = blockIdx.x, cg = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int vpk = t.value_heads / t.key_heads, hk = hv / vpk;
  const int key = t.key_heads * kD, val = t.value_heads * kD, conv = 2 * key + val;
  const float* proj = t.proj + (int64_t)b * t.proj_ld;
  const float* cin = t.conv_in + (int64_t)b * conv * (kKW - 1);
  float* cout = t.conv_out + (int64_t)b * conv * (kKW - 1);
  const bf16* conv_w = (const bf16*)t.conv_w;
  __shared__ float q_s[kD], k_s[kD], v_s[kCols], red[2][kCols];
  const int col = tid % kCols, half = tid / kCols, dv = cg * kCols + col;
  // ---- the prologue's inputs first (loads retire in order, so the conv below
  // then waits only for these while the state streams in behind them): lane l
  // convolves q[l], q[l + 64], k[l], k[l + 64] and, below kCols, one v channel
  constexpr int kCh = 5;
  int ch[kCh];
  float win[kCh][kKW - 1], cw[kCh][kKW], ent[kCh];
#pragma unroll
  for (int j = 0; j < kCh; ++j) {
    ch[j] = j < 4 ? (j < 2 ? 0 : key) + hk * kD + tid + (j & 1) * 64
                  : 2 * key + hv * kD + cg * kCols + (tid < kCols ? tid : 0);
    const float* wp = cin + (int64_t)ch[j] * (kKW - 1);
    const bf16* cwp = conv_w + (int64_t)ch[j] * kKW;
#pragma unroll
    for (int q = 0; q < kKW - 1; ++q) win[j][q] = wp[q];
#pragma unroll
    for (int q = 0; q < kKW; ++q) cw[j][q] = bf2f(cwp[q]);
    ent[j] = proj[ch[j]];
  }
  const float braw = proj[conv + val + hv];
  const float araw = proj[conv + val + t.value_heads + hv];
  const float alog = bf2f(((const bf16*)t.a_log)[hv]), dtb = bf2f(((const bf16*)t.dt_bias)[hv]);
  __builtin_amdgcn_sched_barrier(0);
  float* st = t.state + (((int64_t)b * t.value_heads + hv) * kD + half * kRows) * kD + dv;
  float s[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) s[r] = st[(int64_t)r * kD];
  __builtin_amdgcn_sched_barrier(0);
  // ---- conv + SiLU (conv_silu_f32's arithmetic); the q/k windows advance in the
  // first value head's first group, each v window in the group that owns it
  const bool qk_writer = hv % vpk == 0 && cg == 0;
  float cvv[kCh];
#pragma unroll
  for (int j = 0; j < kCh; ++j) {
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < kKW - 1; ++q) acc += win[j][q] * cw[j][q];
    acc += ent[j] * cw[j][kKW - 1];
    cvv[j] = silu_f(acc);
    if (j < 4 ? qk_writer : tid < kCols) {
      float* o = cout + (int64_t)ch[j] * (kKW - 1);
#pragma unroll
      for (int q = 0; q < kKW - 2; ++q) o[q] = win[j][q + 1];
      o[kKW - 2] = ent[j];
    }
  }
  const float qk[4] = {cvv[0], cvv[1], cvv[2], cvv[3]};
  if (tid < kCols) v_s[tid] = cvv[4];
  // ---- l2 norms (tfd_gdn_step: each 64-value half's wave sum, in order), beta, g
  float sq = 0.f, sk = 0.f;
  sq += wave_sum(qk[0] * qk[0]);
  sq += wave_sum(qk[1] * qk[1]);
  sk += wave_sum(qk[2] * qk[2]);
  sk += wave_sum(qk[3] * qk[3]);
  const float rq = rsqrtf(sq + t.l2_eps), rk = rsqrtf(sk + t.l2_eps);
  const float beta = sigmoid_f(braw);
  const float decay = expf(-expf(alog) * softplus_f(araw + dtb));
  q_s[tid] = qk[0] * (rq * rsqrtf((float)kD));
  q_s[tid + 64] = qk[1] * (rq * rsqrtf((float)kD));
  k_s[tid] = qk[2] * rk;
  k_s[tid + 64] = qk[3] * rk;
  __syncthreads();
  // ---- the delta rule over this thread's half of the key rows
  float rec = 0.f;
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    s[r] *= decay;
    rec += s[r] * k_s[half * kRows + r];
  }
  red[half][col] = rec;
  __syncthreads();
  const float delta = (v_s[col] - (red[0][col] + red[1][col])) * beta;
  float rd = 0.f;
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const float u = s[r] + k_s[half * kRows + r] * delta;
    st[(int64_t)r * kD] = u;
    rd += u * q_s[half * kRows + r];
  }
  __syncthreads();                      // red is reused
  red[half][col] = rd;
  __syncthreads();
  if (half == 0) read[(int64_t)b * ldr + hv * kD + dv] = red[0][col] + red[1][col];
}

// ---------------------------------------------------------------------------
// Experts for rows <= 4 (bf16 weights, the C4 policy).  gate/up: block
// (row tile, slot); slot 0 is the shared expert for every row, slot
// 1 + b k + s the s-th pick of row b.  Each wave routes row b itself
// (route_core: the batched router's arithmetic) and takes pick s; the first
// block of each row's first pick also writes the row's weights and ids.  The
// dot products are those of the grouped gate/up kernel (lanes hold chunks
// c = lane + 64 i), so the SwiGLU vectors agree with it bit for bit.
// ---------------------------------------------------------------------------
template <int kCH, int kR>
__global__ __launch_bounds__(kBlock) void k_moe_small_gateup(TfdMoeArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave);
  const int y = blockIdx.y;
  const bool shared = y == 0;
  const int b = shared ? 0 : (y - 1) / a.k, s = shared ? a.k : (y - 1) % a.k;
  const int H = a.hidden_size, I = shared ? a.shared_inter : a.inter;
  const bf16* xb = (const bf16*)a.x;
  // the expert first: its rows are requested before anything else (loads
  // retire in order, and every wave of the launch reads the same few lines of
  // x, which would hold the weight requests back)
  int e = 0;
  if (!shared) {
    if (a.route == TFD_MOE_ROUTE_SOFTMAX_TOPK) {
      float w;
      int id;
      route_core<0>(a.logits + (int64_t)b * a.ldl, a.experts, a.k, lane, w, id);
      e = __builtin_amdgcn_readlane(id, s);
      if (s == 0 && blockIdx.x == 0 && wave == 0 && lane < a.k) {
        ((float*)a.weights)[(int64_t)b * a.k + lane] = w;
        ((int*)a.idx)[(int64_t)b * a.k + lane] = id;
      }
    } else {
      e = a.idx[(int64_t)b * a.k + s];
    }
    if (e < 0 || e >= a.experts) {
      if (lane == 0) raise_error(a.err, kErrTokenRange);
      e = 0;
    }
  }
  const int r0 = (blockIdx.x * kWavesPerBlock + wave) * kR;
  const bf16* wg = (const bf16*)(shared ? a.w_shared_in : a.w_gate);
  const bf16* wu = (const bf16*)(shared ? a.w_shared_in : a.w_up);
  const int64_t gb = shared ? 0 : (int64_t)e * I;
  const int64_t ub = shared ? I : (int64_t)e * I;
  u32x4 gw[kR][kCH], uw[kR][kCH];
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    const int row = r0 + r < I ? r0 + r : I - 1;
#pragma unroll
    for (int i = 0; i < kCH; ++i) {
      gw[r][i] = WChunk<false>::load(wg, gb + row, H, lane + kWave * i);
      uw[r][i] = WChunk<false>::load(wu, ub + row, H, lane + kWave * i);
    }
  }
  u32x4 xr[kSmallRows][kCH];
#pragma unroll
  for (int r = 0; r < kSmallRows; ++r) {
    const int rr = shared ? (r < a.rows ? r : 0) : b;
    if (shared || r == 0) load_vec<kCH>(xb + (int64_t)rr * H, H, lane, xr[r]);
  }
  if (shared && a.w_shared_scale && blockIdx.x == 0 && wave == 0) {
#pragma unroll
    for (int r = 0; r < kSmallRows; ++r) {      // unrolled: xr stays in registers
      if (r >= a.rows) break;
      const float d = rbf(row_dot<false, kCH>(a.w_shared_scale, 0, H, xr[r], lane));
      if (lane == 0) a.shared_scale[r] = sigmoid_f(d);
    }
  }
  if (r0 >= I) return;
#pragma unroll
  for (int q = 0; q < kSmallRows; ++q) {
    if (shared ? q >= a.rows : q > 0) break;
    const int bb = shared ? q : b;
    bf16* hrow = (bf16*)a.hidden + ((int64_t)bb * (a.k + 1) + s) * a.hidden_ld;
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      float gv = 0.f, uv = 0.f;
#pragma unroll
      for (int i = 0; i < kCH; ++i) {
        gv = dot8(gw[r][i], xr[q][i], gv);
        uv = dot8(uw[r][i], xr[q][i], uv);
      }
      gv = rbf(wave_sum(gv));
      uv = rbf(wave_sum(uv));
      if (lane == 0 && r0 + r < I) hrow[r0 + r] = f2bf(silu_f(gv) * uv);
    }
  }
}

// down + mix: a wave's four 16-lane groups own four output rows n; for row b
// every slot's down row (the picked experts', then the shared expert's) is
// requested at once, each dotted with that slot's SwiGLU vector from LDS (the
// grouped down kernel's lanes and sums), and the slots are mixed in slot order
// with the routing weights and the shared expert's gate, as the mix kernel
// does; the sum goes into the f32 stream.
template <int kCI, int kSlots>
__global__ __launch_bounds__(2 * kWave) void k_moe_small_down(TfdMoeArgs a) {
  constexpr int kLanes = 16, kWaves = 2;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave);
  const int li = lane % kLanes, rsub = lane / kLanes;
  const int H = a.hidden_size, I = a.inter, k = a.k;
  const int n = (blockIdx.x * kWaves + wave) * (kWave / kLanes) + rsub;
  const int nrow = n < H ? n : H - 1;
  __shared__ u32x4 hs[kSlots][kCI * kLanes];
  for (int bb = 0; bb < a.rows; ++bb) {
    // the row's expert ids, then the down rows they select, then the SwiGLU
    // vectors, routing weights, gate and the stream's value (loads retire in
    // order: the weight requests wait only for the ids)
    int ids[kSlots - 1];
#pragma unroll
    for (int q = 0; q < kSlots - 1; ++q) {
      ids[q] = q < k ? a.idx[(int64_t)bb * k + q] : 0;
      ids[q] = ids[q] >= 0 && ids[q] < a.experts ? ids[q] : 0;
    }
    __builtin_amdgcn_sched_barrier(0);
    u32x4 dw[kSlots][kCI];
#pragma unroll
    for (int q = 0; q < kSlots; ++q) {
      const bool sh = q == kSlots - 1;
      const bf16* w = (const bf16*)(sh ? a.w_shared_out : a.w_down);
      const int64_t row = sh ? nrow : (int64_t)ids[q] * H + nrow;
      if (sh || q < k) {
#pragma unroll
        for (int i = 0; i < kCI; ++i) dw[q][i] = WChunk<false>::load(w, row, I, li + kLanes * i);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    const bf16* hb = (const bf16*)a.hidden + (int64_t)bb * (k + 1) * a.hidden_ld;
    u32x4 hv[(kSlots * kCI * kLanes + 2 * kWave - 1) / (2 * kWave)];
#pragma unroll
    for (int j = 0; j < (int)(sizeof(hv) / sizeof(hv[0])); ++j) {
      const int q = threadIdx.x + 2 * kWave * j, slot = q / (kCI * kLanes), c = q % (kCI * kLanes);
      hv[j] = slot <= k ? load16(hb + (int64_t)slot * a.hidden_ld + 8 * c) : u32x4{0u, 0u, 0u, 0u};
    }
    float wts[kSlots - 1];
#pragma unroll
    for (int q = 0; q < kSlots - 1; ++q) wts[q] = q < k ? a.weights[(int64_t)bb * k + q] : 0.f;
    const float sscale = a.w_shared_scale ? a.shared_scale[bb] : 1.f;
    const float prev = a.accumulate ? a.out[(int64_t)bb * H + nrow] : 0.f;   // the stream's value
    __syncthreads();                    // the previous row's vectors are read
#pragma unroll
    for (int j = 0; j < (int)(sizeof(hv) / sizeof(hv[0])); ++j) {
      const int q = threadIdx.x + 2 * kWave * j, slot = q / (kCI * kLanes), c = q % (kCI * kLanes);
      if (slot < kSlots) hs[slot][c] = hv[j];
    }
    __syncthreads();
    float d[kSlots];
#pragma unroll
    for (int q = 0; q < kSlots; ++q) {
      const bool sh = q == kSlots - 1;
      const int hslot = sh ? k : q;
      float acc = 0.f;
      if (sh || q < k) {
#pragma unroll
        for (int i = 0; i < kCI; ++i) acc = dot8(dw[q][i], hs[hslot][li + kLanes * i], acc);
      }
      d[q] = rbf(group_sum<kLanes>(acc));
    }
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < kSlots - 1; ++q)
      if (q < k) acc += d[q] * wts[q];
    const float yv = acc + d[kSlots - 1] * sscale;
    if (li == 0 && n < H) a.out[(int64_t)bb * H + n] = a.accumulate ? prev + yv : yv;
  }
}

}  // namespace

extern "C" {

int tfd_rowgemv_bf16(const TfdRowGemvArgs* args, void* stream) {
  if (!args) return fail(kBadArg, "rowgemv: null args");
  const TfdRowGemvArgs& a = *args;
  if (!a.x || !a.w || !a.out) return fail(kBadArg, "rowgemv: null pointer");
  if (a.rows < 1 || a.rows > kSmallRows || (a.K != 2048 && a.K != 4096) || a.N < 1 ||
      a.ldo < a.N)
    return fail(kBadShape, "rowgemv: rows=%d (1..%d) K=%d (2048 or 4096) N=%d ldo=%d", a.rows,
                kSmallRows, a.K, a.N, a.ldo);
  if (a.epilogue != TFD_EPI_LOGITS && a.epilogue != TFD_EPI_RESID_F32)
    return fail(kBadArg, "rowgemv: epilogue %d (logits or resid_f32)", a.epilogue);
  switch (a.x_kind) {
    case TFD_ROWX_NORM_F32:
      if (!a.gamma || a.ldx < a.K) return fail(kBadArg, "rowgemv: norm needs gamma, ldx >= K");
      break;
    case TFD_ROWX_GATED_F32:
      if (!a.gamma || !a.gate || a.head_dim != 128 || a.ldx < a.K || a.ldg < a.K)
        return fail(kBadArg, "rowgemv: gated norm needs gamma, gate, head_dim 128, ldx/ldg >= K");
      break;
    case TFD_ROWX_OPERAND:
      break;
    case TFD_ROWX_ROWS:
      if (a.ldx < a.K) return fail(kBadShape, "rowgemv: ldx < K");
      break;
    default:
      return fail(kBadArg, "rowgemv: x_kind %d", a.x_kind);
  }
  if (a.x_rows && a.ldxr < a.K) return fail(kBadShape, "rowgemv: ldxr < K");
  // a short normed projection (the router: 256 rows) takes one row per wave,
  // four times the blocks and a quarter of the loads in flight per lane; every
  // row's sum is the same whichever wave makes it
  const bool one_row = a.K == 2048 && a.N <= 512 && a.x_kind == TFD_ROWX_NORM_F32;
  const int kG = a.K == 2048 ? (one_row ? 1 : 4) : 2;
  const int ngroups = (a.N + kG - 1) / kG;
  const int blocks = std::min((ngroups + kWavesPerBlock - 1) / kWavesPerBlock, 2048);
  hipStream_t s = (hipStream_t)stream;
#define TFD_RG(X, E, C, G) \
  hipLaunchKernelGGL((k_rowgemv<X, E, C, G>), dim3(blocks), dim3(kBlock), 0, s, a)
#define TFD_RG_E(X, C, G)                                   \
  do {                                                      \
    if (a.epilogue == TFD_EPI_LOGITS) TFD_RG(X, TFD_EPI_LOGITS, C, G); \
    else TFD_RG(X, TFD_EPI_RESID_F32, C, G);               \
  } while (0)
#define TFD_RG_K(X)                        \
  do {                                     \
    if (a.K == 2048) TFD_RG_E(X, 4, 4);    \
    else TFD_RG_E(X, 8, 2);                \
  } while (0)
  switch (a.x_kind) {
    case TFD_ROWX_NORM_F32:
      if (one_row) TFD_RG_E(TFD_ROWX_NORM_F32, 4, 1);
      else TFD_RG_K(TFD_ROWX_NORM_F32);
      break;
    case TFD_ROWX_GATED_F32: TFD_RG_K(TFD_ROWX_GATED_F32); break;
    case TFD_ROWX_OPERAND: TFD_RG_K(TFD_ROWX_OPERAND); break;
    default: TFD_RG_K(TFD_ROWX_ROWS); break;
  }
#undef TFD_RG_K
#undef TFD_RG_E
#undef TFD_RG
  return launched("rowgemv");
}

int tfd_gdn_step_cols(const TfdGdnArgs* args, float* read, int ldr, void* stream) {
  if (!args || !read) return fail(kBadArg, "gdn_step_cols: null args");
  const TfdGdnArgs& t = *args;
  if (!t.proj || !t.conv_in || !t.conv_out || !t.state || !t.conv_w || !t.a_log ||
      !t.dt_bias || t.conv_in == t.conv_out)
    return fail(kBadArg, "gdn_step_cols: null pointer, or conv_out == conv_in");
  if (t.rows <= 0 || t.rows > 32 || t.head_k_dim != 128 || t.head_v_dim != 128 ||
      t.key_heads <= 0 || t.value_heads % t.key_heads || t.conv_kernel != 4 ||
      t.proj_ld < 2 * t.key_heads * 128 + 2 * t.value_heads * 128 + 2 * t.value_heads ||
      ldr < t.value_heads * 128)
    return fail(kBadShape, "gdn_step_cols: rows=%d (1..32) dk=%d dv=%d (128) hk=%d hv=%d kw=%d "
                "ldr=%d", t.rows, t.head_k_dim, t.head_v_dim, t.key_heads, t.value_heads,
                t.conv_kernel, ldr);
  constexpr int kCols = 32;
  hipLaunchKernelGGL(k_gdn_cols<kCols>, dim3(t.value_heads, 128 / kCols, t.rows),
                     dim3(2 * kCols), 0, (hipStream_t)stream, t, read, ldr);
  return launched("gdn_step_cols");
}

int tfd_moe_experts_small(const TfdMoeArgs* args, void* stream) {
  if (!args) return fail(kBadArg, "moe_small: null args");
  const TfdMoeArgs& a = *args;
  if (!a.x || !a.weights || !a.idx || !a.w_gate || !a.w_up || !a.w_down || !a.w_shared_in ||
      !a.w_shared_out || !a.hidden || !a.out || (a.w_shared_scale && !a.shared_scale))
    return fail(kBadArg, "moe_small: null pointer");
  if (a.fp8 || a.policy != TFD_POLICY_F32 || a.resid)
    return fail(kUnsupported, "moe_small: bf16 weights and the f32 policy only");
  if (a.route != TFD_MOE_ROUTE_GIVEN && a.route != TFD_MOE_ROUTE_SOFTMAX_TOPK)
    return fail(kUnsupported, "moe_small: routing %d", a.route);
  if (a.route == TFD_MOE_ROUTE_SOFTMAX_TOPK && (!a.logits || a.ldl < a.experts))
    return fail(kBadArg, "moe_small: routing needs logits with ldl >= experts");
  if (a.rows < 1 || a.rows > kSmallRows || a.hidden_size != 2048 || a.inter != 512 ||
      a.shared_inter != 512 || a.hidden_ld < 512 || a.k < 1 || a.k > 8 || a.experts < a.k ||
      a.experts > 256)
    return fail(kBadShape, "moe_small: rows=%d (1..%d) hidden=%d (2048) inter=%d shared=%d (512) "
                "k=%d (1..8) experts=%d (<= 256)", a.rows, kSmallRows, a.hidden_size, a.inter,
                a.shared_inter, a.k, a.experts);
  hipStream_t s = (hipStream_t)stream;
  constexpr int kR = 2;
  hipLaunchKernelGGL((k_moe_small_gateup<4, kR>), dim3(512 / (kWavesPerBlock * kR),
                     1 + a.rows * a.k), dim3(kBlock), 0, s, a);
  hipLaunchKernelGGL((k_moe_small_down<4, 9>), dim3(2048 / (2 * 4)), dim3(2 * kWave), 0, s, a);
  return launched("moe_experts_small");
}

}  // extern "C"
