// Decode-step pieces of the hybrid models, for gfx950: the MoE routers and
// experts, the gated-DeltaNet recurrence (Qwen3.5, workload C4) and the Mamba2
// recurrence (Granite-4.0-H, workload C5).
//
// Arithmetic policies (one per model, the one its reference states):
//  * C4 follows the example's plain-torch twin (torch_ref.py's dtype policy):
//    f32 activations and f32 recurrent state; a matmul's activation is cast to
//    bf16, summed in f32 and the result rounded to bf16 once.
//  * C5 follows the authored HIR: bf16 activations with every binary op
//    rounded, f32 where the HIR casts to f32, f32 SSM state; weights are
//    fp8-e4m3fn with one f32 scale per output channel.
// Batch rows are sequences (one token each); the projections around these
// kernels are the skinny GEMMs (tfd_gemm_skinny_bf16 / _fp8).

#include "hybrid_common.h"
#include "host_common.h"
#include "tf_decode.h"
#include "tf_hybrid.h"

#include <type_traits>

using namespace tfd;
using namespace tfd_host;
using namespace tfd_hybrid;

namespace {

typedef float f32x2_t __attribute__((ext_vector_type(2)));

constexpr int kMaxRowsH = 32;

template <int kMode>
__global__ __launch_bounds__(kWave) void k_route(const float* __restrict__ logits, int ldl, int E,
                                                 int k, float* __restrict__ weights,
                                                 int* __restrict__ idx) {
  const int row = blockIdx.x;
  route_row<kMode>(logits + (int64_t)row * ldl, E, k, weights + (int64_t)row * k,
                   idx + (int64_t)row * k, threadIdx.x);
}

// ---------------------------------------------------------------------------
// Experts, grouped by expert: every weight row of an expert some sequence
// picked is read once per launch, whatever the number of sequences that picked
// it.  A lane holds 16-byte chunks of the bf16 input (8 values) and the
// matching 8 weights of a row (bf16, or fp8 with one scale per row); exact
// products are summed in f32 and the wave adds its lanes.
//   group   one block: expert -> its (sequence, slot) entries, and the list of
//           the experts picked at all (ascending)
//   gate/up (picked expert or the shared one) x (row tile): a wave keeps kR
//           gate rows and kR up rows in registers and runs every entry of the
//           expert through them -> the SwiGLU hidden vector of each entry
//   down    the same over the down projections -> one bf16-rounded output
//           vector per (sequence, slot)
//   mix     per sequence, the slots in slot order, then the shared expert
// ---------------------------------------------------------------------------
struct MoeArgs {
  const bf16* x;            // [B][H] the normalised tokens
  const float* weights;     // [B][k] routing weights
  const int* idx;           // [B][k] expert ids
  const void *w_gate, *w_up, *w_down;        // [E][I][H], [E][I][H], [E][H][I]
  const float *s_gate, *s_up, *s_down;       // fp8 row scales [E][I], [E][I], [E][H]
  const void *w_sin, *w_sout;                // shared: [2 IS][H] (gate rows, then up), [H][IS]
  const float *s_sin, *s_sout;               // fp8 row scales [2 IS], [H]
  const bf16* w_sscale;                      // C4 shared-expert gate row [H] (or null)
  bf16* hidden;                              // [B][k + 1][IM] work: SwiGLU vectors
  float* sscale;                             // [B] work: the shared expert's sigmoid gate
  float* partial;                            // [B][k + 1][H] work: down outputs per slot
  int* groups;                               // work: n | picked[E] | count[E] | entries[E][B]
  float* out;                                // [B][H]
  const float* logits;                       // [B][ldl] router logits when route >= 0
  int ldl, route;                            // route: -1 given weights/idx, else mode
  int B, H, I, IS, IM, k, E;
  int accumulate;                            // out += (f32 policy)
  bf16* resid;                               // bf16 policy: resid = bf16(resid + bf16(y m))
  float resid_mult;
  int* err;
};

__device__ __forceinline__ int* grp_picked(const MoeArgs& a) { return a.groups + 1; }
__device__ __forceinline__ int* grp_count(const MoeArgs& a) { return a.groups + 1 + a.E; }
__device__ __forceinline__ int* grp_entries(const MoeArgs& a) { return a.groups + 1 + 2 * a.E; }

// One block: (optionally) route every row, one wave per row, then group.
constexpr int kGroupThreads = 1024;
constexpr int kMaxExperts = 256;
template <int kRoute>
__global__ __launch_bounds__(kGroupThreads) void k_moe_group(MoeArgs a) {
  constexpr int kWaves = kGroupThreads / kWave;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  __shared__ int c_s[kMaxExperts];
  __shared__ int wave_n[kWaves];
  if (kRoute >= 0) {
    // the routing outputs are this call's weights and ids
    for (int r = wave; r < a.B; r += kWaves)
      route_row<kRoute>(a.logits + (int64_t)r * a.ldl, a.E, a.k,
                        const_cast<float*>(a.weights) + (int64_t)r * a.k,
                        const_cast<int*>(a.idx) + (int64_t)r * a.k, lane);
  }
  if (tid < kMaxExperts) c_s[tid] = 0;
  __syncthreads();
  int* entries = grp_entries(a);
  for (int i = tid; i < a.B * a.k; i += kGroupThreads) {
    int e = a.idx[i];
    if (e < 0 || e >= a.E) {
      raise_error(a.err, kErrTokenRange);
      e = 0;
    }
    const int p = atomicAdd(&c_s[e], 1);
    if (p < a.B)
      entries[(int64_t)e * a.B + p] = i;
    else
      raise_error(a.err, kErrTokenRange);   // an expert picked twice by one sequence
  }
  __syncthreads();
  const int e = tid;
  const bool on = e < a.E && c_s[e] > 0;
  const uint64_t m = __ballot(on);
  if (lane == 0) wave_n[wave] = __popcll(m);
  __syncthreads();
  int off = 0;
  for (int w = 0; w < wave; ++w) off += wave_n[w];
  if (on) grp_picked(a)[off + __popcll(m & ((1ull << lane) - 1ull))] = e;
  if (e < a.E) grp_count(a)[e] = c_s[e] < a.B ? c_s[e] : a.B;
  if (tid == 0) {
    int n = 0;
    for (int w = 0; w < kWaves; ++w) n += wave_n[w];
    a.groups[0] = n;
  }
}

// (expert, entries) of blockIdx.y: the shared expert, then the picked ones.
// The shared expert has an entry per sequence (its blocks loop longest), so it
// comes first in dispatch order and overlaps the picked experts instead of
// trailing them.  kWho selects what a launch covers: 0 both (the shared expert
// is y = 0),
// 1 the picked experts only, 2 the shared expert only (when its width differs
// from the routed experts', each gets a launch sized for it).
struct Group {
  bool shared;
  int e, count;
  const int* entries;
};
template <int kWho>
__device__ __forceinline__ bool moe_group(const MoeArgs& a, Group& g) {
  g.shared = kWho == 2 || (kWho == 0 && blockIdx.y == 0);
  if (g.shared) {
    g.e = 0;
    g.count = a.B;
    g.entries = nullptr;
    return true;
  }
  const int y = kWho == 0 ? (int)blockIdx.y - 1 : (int)blockIdx.y;
  if (y >= a.groups[0]) return false;
  g.e = grp_picked(a)[y];
  g.count = grp_count(a)[g.e];
  g.entries = grp_entries(a) + (int64_t)g.e * a.B;
  return true;
}
// sequence and slot of entry t of the group (slot k: the shared expert)
__device__ __forceinline__ void moe_entry(const MoeArgs& a, const Group& g, int t, int& b,
                                          int& slot) {
  if (g.shared) {
    b = t;
    slot = a.k;
  } else {
    const int i = g.entries[t];
    b = i / a.k;
    slot = i % a.k;
  }
}

template <bool kFp8, bool kF32, int kC, int kR, int kWho = 0>
__global__ __launch_bounds__(kBlock) void k_moe_gateup(MoeArgs a) {
  using WC = WChunk<kFp8>;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  Group g;
  if (!moe_group<kWho>(a, g)) return;
  if (g.shared && a.w_sscale && blockIdx.x == 0 && wave == 0) {
    for (int b = 0; b < a.B; ++b) {
      u32x4 xr[kC];
      load_vec<kC>(a.x + (int64_t)b * a.H, a.H, lane, xr);
      const float d = rbf(row_dot<false, kC>(a.w_sscale, 0, a.H, xr, lane));
      if (lane == 0) a.sscale[b] = sigmoid_f(d);
    }
  }
  const int nrows = g.shared ? a.IS : a.I;
  const int r0 = (blockIdx.x * kWavesPerBlock + wave) * kR;
  if (r0 >= nrows) return;
  const void* wg = g.shared ? a.w_sin : a.w_gate;
  const void* wu = g.shared ? a.w_sin : a.w_up;
  const int64_t gb = g.shared ? 0 : (int64_t)g.e * a.I;
  const int64_t ub = g.shared ? a.IS : (int64_t)g.e * a.I;
  const int nch = a.H / 8;
  typename WC::T gw[kR][kC], uw[kR][kC];
  float gs[kR], us[kR];
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    const int row = r0 + r < nrows ? r0 + r : nrows - 1;
#pragma unroll
    for (int i = 0; i < kC; ++i) {
      const int c = lane + kWave * i < nch ? lane + kWave * i : 0;
      gw[r][i] = WC::load(wg, gb + row, a.H, c);
      uw[r][i] = WC::load(wu, ub + row, a.H, c);
    }
    if (kFp8) {
      gs[r] = g.shared ? a.s_sin[row] : a.s_gate[gb + row];
      us[r] = g.shared ? a.s_sin[a.IS + row] : a.s_up[gb + row];
    }
  }
  for (int t = 0; t < g.count; ++t) {
    int b, slot;
    moe_entry(a, g, t, b, slot);
    u32x4 xr[kC];
    load_vec<kC>(a.x + (int64_t)b * a.H, a.H, lane, xr);
    bf16* hrow = a.hidden + ((int64_t)b * (a.k + 1) + slot) * a.IM;
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      float gv = 0.f, uv = 0.f;
#pragma unroll
      for (int i = 0; i < kC; ++i) {
        if (lane + kWave * i < nch) {
          gv = WC::dot(gw[r][i], xr[i], gv);
          uv = WC::dot(uw[r][i], xr[i], uv);
        }
      }
      gv = wave_sum(gv);
      uv = wave_sum(uv);
      if (kFp8) {
        gv *= gs[r];
        uv *= us[r];
      }
      gv = rbf(gv);
      uv = rbf(uv);
      const float h = kF32 ? silu_f(gv) * uv : rbf(silu_f(gv)) * uv;
      if (lane == 0 && r0 + r < nrows) hrow[r0 + r] = f2bf(h);
    }
  }
}

// The down projections are short rows (K = the expert width): sixteen lanes
// share a row (16-byte chunks c = l % 16 + 16 i), a wave holds four rows per
// pass and kP passes, and a row's sum needs only the in-row DPP steps.
constexpr int kDownLanes = 16;
template <bool kFp8, int kC, int kP, int kWho = 0>
__global__ __launch_bounds__(kBlock) void k_moe_down(MoeArgs a) {
  using WC = WChunk<kFp8>;
  constexpr int kRpp = kWave / kDownLanes;        // rows per pass
  constexpr int kR = kRpp * kP;                   // rows per wave
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int li = lane % kDownLanes, rsub = lane / kDownLanes;
  Group g;
  if (!moe_group<kWho>(a, g)) return;
  const int K = g.shared ? a.IS : a.I;
  const int nch = K / 8;
  const int n0 = (blockIdx.x * kWavesPerBlock + wave) * kR;
  if (n0 >= a.H) return;
  const void* w = g.shared ? a.w_sout : a.w_down;
  const int64_t base = g.shared ? 0 : (int64_t)g.e * a.H;
  typename WC::T dw[kP][kC];
  float ds[kP];
#pragma unroll
  for (int p = 0; p < kP; ++p) {
    const int n = n0 + p * kRpp + rsub;
    const int row = n < a.H ? n : a.H - 1;
#pragma unroll
    for (int i = 0; i < kC; ++i) {
      const int c = li + kDownLanes * i < nch ? li + kDownLanes * i : 0;
      dw[p][i] = WC::load(w, base + row, K, c);
    }
    if (kFp8) ds[p] = g.shared ? a.s_sout[row] : a.s_down[base + row];
  }
  // entry t's SwiGLU vector, and its products into its partial row
  auto hload = [&](int t, u32x4 (&hr)[kC]) {
    int b, slot;
    moe_entry(a, g, t, b, slot);
    const bf16* hv = a.hidden + ((int64_t)b * (a.k + 1) + slot) * a.IM;
#pragma unroll
    for (int i = 0; i < kC; ++i) {
      const int c = li + kDownLanes * i;
      hr[i] = c < nch ? load16(hv + (int64_t)c * 8) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto products = [&](int t, const u32x4 (&hr)[kC]) {
    int b, slot;
    moe_entry(a, g, t, b, slot);
    float* prow = a.partial + ((int64_t)b * (a.k + 1) + slot) * a.H;
#pragma unroll
    for (int p = 0; p < kP; ++p) {
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < kC; ++i)
        if (li + kDownLanes * i < nch) d = WC::dot(dw[p][i], hr[i], d);
      d = group_sum<kDownLanes>(d);
      if (kFp8) d *= ds[p];
      const int n = n0 + p * kRpp + rsub;
      if (li == 0 && n < a.H) prow[n] = rbf(d);
    }
  };
  if constexpr (kWho == 2) {
    // the shared expert's launch: an entry per sequence, so the next entry's
    // vector is requested before this one's products (the last request
    // repeats the last entry, so every iteration issues the same loads)
    u32x4 hr[kC], hn[kC];
    hload(0, hr);
    for (int t = 0; t < g.count; ++t) {
      hload(t + 1 < g.count ? t + 1 : t, hn);
      products(t, hr);
#pragma unroll
      for (int i = 0; i < kC; ++i) hr[i] = hn[i];
    }
  } else {
    for (int t = 0; t < g.count; ++t) {
      u32x4 hr[kC];
      hload(t, hr);
      products(t, hr);
    }
  }
}

template <bool kF32>
__global__ __launch_bounds__(kBlock) void k_moe_mix(MoeArgs a) {
  const int b = blockIdx.y, n = blockIdx.x * kBlock + threadIdx.x;
  if (n >= a.H) return;
  const float* pb = a.partial + (int64_t)b * (a.k + 1) * a.H + n;
  const float* wb = a.weights + (int64_t)b * a.k;
  float acc = 0.f;
  constexpr int kBatch = 8;           // a batch's loads are all issued before the adds
  for (int s0 = 0; s0 < a.k; s0 += kBatch) {
    float d[kBatch], wg[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int s = s0 + i < a.k ? s0 + i : a.k - 1;
      d[i] = pb[(int64_t)s * a.H];
      wg[i] = wb[s];
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i)
      if (s0 + i < a.k) acc += kF32 ? d[i] * wg[i] : rbf(d[i] * wg[i]);
  }
  const float dsh = pb[(int64_t)a.k * a.H];
  const int64_t at = (int64_t)b * a.H + n;
  if (kF32) {
    const float y = acc + dsh * (a.w_sscale ? a.sscale[b] : 1.f);
    a.out[at] = a.accumulate ? a.out[at] + y : y;
  } else {
    const float y = rbf(rbf(acc) + dsh);
    if (a.resid)
      a.resid[at] = f2bf(bf2f(a.resid[at]) + rbf(y * a.resid_mult));
    else
      a.out[at] = y;
  }
}

// ---------------------------------------------------------------------------
// Experts for at most 16 sequences, on the matrix cores, over weights packed
// as the skinny GEMMs pack them (tfd_pack_skinny_bf16 / _fp8 of each [rows][K]
// matrix, the experts' matrices stacked: expert e's rows e * I ..).  The
// entries of a group (the sequences that picked its expert) are the rows of
// one 16-row MFMA tile, rows past the count zero, so each (entry, weight row)
// sum stays in the accumulators -- no wave sum per pair -- and every weight
// byte of a picked expert is read once per launch, a wave's load of a 32-wide
// K step being one contiguous packed block.  fp8 codes are decoded to bf16 in
// registers, exactly, as in the skinny GEMMs.  The group lists of k_moe_group
// are staged into LDS first; a wave decodes an item once, when its loads
// reach it, so a step costs its loads, its decode and its MFMAs.
//   gate/up  items of 16 gate + 16 up rows of the shared expert or of a picked
//            one over the whole hidden size, dealt to the blocks in turn; the
//            four waves of a block split K, their sums meet in LDS (two
//            buffers, one barrier per item) and one wave, in turn, writes the
//            SwiGLU of each (entry, row)
//   down     a block per 16 output columns: its waves take the items in turn --
//            the shared expert's K halves of the routed width, then the picked
//            experts -- each a 16-column tile against the hidden vectors of the
//            item's entries, into LDS; then per sequence the slots are mixed in
//            slot order and the result goes into the stream, as k_moe_mix does
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8_m __attribute__((ext_vector_type(8)));
typedef float f32x4_m __attribute__((ext_vector_type(4)));
constexpr int kM8 = 16;          // entries of a group at most: the tile's rows
constexpr int kM8Slots = 17;     // k + 1 at most
constexpr int kM8Depth = 8;      // 32-wide K steps in flight per wave

struct M8Meta {
  int n;                         // experts picked
  int picked[kMaxExperts];
  int count[kMaxExperts];
  uint16_t ent[kMaxExperts][kM8];   // entry t of expert e: (sequence << 8) | slot
};

__device__ __forceinline__ void m8_stage(const MoeArgs& a, M8Meta& m) {
  for (int i = threadIdx.x; i < a.E; i += blockDim.x) {
    m.picked[i] = grp_picked(a)[i];
    m.count[i] = grp_count(a)[i];
  }
  const int* ent = grp_entries(a);
  for (int i = threadIdx.x; i < a.E * a.B; i += blockDim.x) {
    // entries past an expert's count are stale and never read
    const unsigned v = (unsigned)ent[i];
    m.ent[i / a.B][i % a.B] = (uint16_t)((((v / a.k) & 0xffu) << 8) | ((v % a.k) & 0xffu));
  }
  if (threadIdx.x == 0) m.n = a.groups[0];
  __syncthreads();
}

// lane l's B operand of packed block `blk`: W[16 t + l % 16][32 s + 8 (l / 16) .. +7]
template <bool kFp8>
struct M8W {
  using Raw = u32x2;
  static __device__ __forceinline__ Raw load(const void* w, int64_t blk, int lane) {
    return __builtin_nontemporal_load(
        reinterpret_cast<const u32x2*>((const uint8_t*)w + blk * 512 + lane * 8));
  }
  static __device__ __forceinline__ bf16x8_m value(const Raw& r) {
    typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
    const bf16x2_v p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r.x, 1.0f, false);
    const bf16x2_v p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r.x, 1.0f, true);
    const bf16x2_v p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r.y, 1.0f, false);
    const bf16x2_v p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r.y, 1.0f, true);
    return bf16x8_m{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
  }
};
template <>
struct M8W<false> {
  using Raw = u32x4;
  static __device__ __forceinline__ Raw load(const void* w, int64_t blk, int lane) {
    return load16_stream((const bf16*)w + blk * 512 + lane * 8);
  }
  static __device__ __forceinline__ bf16x8_m value(const Raw& r) {
    return __builtin_bit_cast(bf16x8_m, r);
  }
};

// A operands through a range-limited descriptor (rsrc_bounded): a lane whose
// row is past the group's count reads at kM8Off, out of range, which returns
// zeros without a memory access (the rows of the sequences that did not pick
// the expert cost nothing)
constexpr uint32_t kM8Off = kOutOfRange;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t m8_rsrc(const void* base, uint32_t bytes) {
  return rsrc_bounded(base, bytes);
}
__device__ __forceinline__ bf16x8_m m8_a(const u32x4& x) { return __builtin_bit_cast(bf16x8_m, x); }

template <bool kFp8, bool kF32>
__global__ __launch_bounds__(kBlock) void k_moe8_gateup(MoeArgs a) {
  using W = M8W<kFp8>;
  constexpr int kD = kM8Depth;
  __shared__ M8Meta meta;
  __shared__ f32x4_m red[2][kWavesPerBlock][2][kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  if (a.w_sscale && blockIdx.x == gridDim.x - 1 && wave == kWavesPerBlock - 1) {
    // C4's shared-expert gate, sigmoid(bf16(w . x)) per sequence, summed as
    // k_moe_gateup sums it
    for (int b = 0; b < a.B; ++b) {
      const bf16* xr = a.x + (int64_t)b * a.H;
      float acc = 0.f;
      for (int c = lane; c < a.H / 8; c += kWave)
        acc = dot8(load16(a.w_sscale + (int64_t)c * 8), load16(xr + (int64_t)c * 8), acc);
      const float d = rbf(wave_sum(acc));
      if (lane == 0) a.sscale[b] = sigmoid_f(d);
    }
  }
  m8_stage(a, meta);
  const int nS = a.IS / 16, nT = a.I / 16;
  const int items = nS + meta.n * nT;
  const int G = (int)gridDim.x, me = (int)blockIdx.x;
  if (me >= items) return;
  const int mine = (items - 1 - me) / G + 1;
  const int ksteps = a.H / 32;                    // packed blocks per tile
  const int ns = ksteps / kWavesPerBlock;         // this wave's steps per item (>= kD)
  const int k0 = wave * ns;                       // this wave's first step
  const int nl = lane & 15, kq = lane >> 4;       // tile row / A row, K octet of a step
  // an item as its loads see it: the first packed blocks of its gate and up
  // rows for this wave, the A row of this lane and its validity
  struct Item {
    const void *wg, *wu;
    int64_t gblk, ublk;
    uint32_t xo;                                  // this lane's A bytes, or kM8Off
  };
  const auto xrs = m8_rsrc(a.x, (uint32_t)a.B * a.H * 2u);
  auto decode = [&](int j) {
    const int it = me + j * G;
    Item d;
    if (it < nS) {
      d.wg = a.w_sin;
      d.wu = a.w_sin;
      d.gblk = (int64_t)it * ksteps + k0;
      d.ublk = (int64_t)(nS + it) * ksteps + k0;
      d.xo = nl < a.B ? ((uint32_t)nl * a.H + k0 * 32 + kq * 8) * 2u : kM8Off;
    } else {
      const int r = it - nS, e = meta.picked[r / nT];
      const int64_t t = (int64_t)e * nT + r % nT;
      d.wg = a.w_gate;
      d.wu = a.w_up;
      d.gblk = t * ksteps + k0;
      d.ublk = d.gblk;
      d.xo = nl < meta.count[e]
                 ? ((uint32_t)(meta.ent[e][nl] >> 8) * a.H + k0 * 32 + kq * 8) * 2u
                 : kM8Off;
    }
    return d;
  };
  typename W::Raw gw[kD], uw[kD];
  u32x4 xs[kD];
  Item nx = decode(0);
  int jn = 0, sn = 0;                             // the next step to load
  auto issue = [&](int u) {
    gw[u] = W::load(nx.wg, nx.gblk + sn, lane);
    uw[u] = W::load(nx.wu, nx.ublk + sn, lane);
    xs[u] = __builtin_amdgcn_raw_buffer_load_b128(xrs, nx.xo + sn * 64u, 0, 0);
    if (++sn == ns && jn + 1 < mine) {
      sn = 0;
      nx = decode(++jn);
    }
  };
  f32x4_m cg = {0.f, 0.f, 0.f, 0.f}, cu = cg;
  int jc = 0, sc = 0;                             // the step being computed
  auto compute = [&](int u) {
    const bf16x8_m x = m8_a(xs[u]);
    cg = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, W::value(gw[u]), cg, 0, 0, 0);
    cu = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, W::value(uw[u]), cu, 0, 0, 0);
    if (++sc < ns) return;
    // item jc done: the four K quarters meet in LDS, one wave writes the rows
    const int j = jc++;
    sc = 0;
    red[j & 1][wave][0][lane] = cg;
    red[j & 1][wave][1][lane] = cu;
    cg = f32x4_m{0.f, 0.f, 0.f, 0.f};
    cu = cg;
    __syncthreads();
    if (wave != (j & (kWavesPerBlock - 1))) return;
    const int it = me + j * G;
    const bool sh = it < nS;
    const int r = it - nS, e = sh ? 0 : meta.picked[r / nT];
    const int cnt = sh ? a.B : meta.count[e];
    const int row = (sh ? it : r % nT) * 16 + nl;
    const int64_t grow = sh ? row : (int64_t)e * a.I + row;
    const int64_t urow = sh ? (int64_t)a.IS + row : grow;
    float gs = 1.f, us = 1.f;
    if (kFp8) {
      gs = sh ? a.s_sin[grow] : a.s_gate[grow];
      us = sh ? a.s_sin[urow] : a.s_up[urow];
    }
    f32x4_m sg = red[j & 1][0][0][lane], su = red[j & 1][0][1][lane];
#pragma unroll
    for (int w = 1; w < kWavesPerBlock; ++w) {
      const f32x4_m vg = red[j & 1][w][0][lane], vu = red[j & 1][w][1][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sg[i] += vg[i];
        su[i] += vu[i];
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 4 * kq + i;
      if (m >= cnt) continue;
      const int bs = sh ? (m << 8) | a.k : meta.ent[e][m];
      float gv = sg[i], uv = su[i];
      if (kFp8) {
        gv *= gs;
        uv *= us;
      }
      gv = rbf(gv);
      uv = rbf(uv);
      const float h = kF32 ? silu_f(gv) * uv : rbf(silu_f(gv)) * uv;
      a.hidden[((int64_t)(bs >> 8) * (a.k + 1) + (bs & 0xff)) * a.IM + row] = f2bf(h);
    }
  };
  const int total = mine * ns;                    // a multiple of kD
#pragma unroll
  for (int u = 0; u < kD; ++u) issue(u);
  int q0 = 0;
  for (; q0 + kD < total; q0 += kD) {
#pragma unroll
    for (int u = 0; u < kD; ++u) {
      compute(u);
      issue(u);
    }
  }
#pragma unroll
  for (int u = 0; u < kD; ++u) compute(u);
}

// The down kernel's units: kM8Depth 32-wide steps (256 of K) of one item, so
// every unit is as long as every other and the waves of a block finish
// together; each unit's sums have their own place in LDS and the mix adds a
// slot's units in K order.
constexpr int kM8Unit = 32 * kM8Depth;
constexpr int kM8Parts = 1024;       // (sequence, slot, unit) sums of the routed experts
constexpr int kM8SharedUnits = 8;    // units of the shared expert's width

template <bool kFp8, bool kF32, int kWv, int kD = kM8Depth>
__global__ __launch_bounds__(kWv * kWave) void k_moe8_down(MoeArgs a) {
  using W = M8W<kFp8>;
  constexpr int kUnit = 32 * kD;                  // K of a unit
  __shared__ M8Meta meta;
  __shared__ float part[kM8Parts * 16];              // [sequence][slot][unit][column]
  __shared__ float shp[kM8SharedUnits * kM8 * 16];   // [unit][sequence][column]
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int nl = lane & 15, kq = lane >> 4;
  const int ct = (int)blockIdx.x;                 // 16-column tile of the output
  const int uS = a.IS / kUnit, uR = a.I / kUnit;
  struct Unit {
    const void* w;
    int64_t blk;
    uint32_t ho;                                  // this lane's A bytes, or kM8Off
  };
  const auto hrs = m8_rsrc(a.hidden, (uint32_t)a.B * (a.k + 1) * a.IM * 2u);
  auto decode = [&](int j) {
    const int u = wave + j * kWv;
    Unit d;
    if (u < uS) {
      d.w = a.w_sout;
      d.blk = (int64_t)ct * (a.IS / 32) + u * kD;
      d.ho = nl < a.B ? (((uint32_t)nl * (a.k + 1) + a.k) * a.IM + u * kUnit + kq * 8) * 2u
                      : kM8Off;
    } else {
      const int r = u - uS, e = meta.picked[r / uR], pt = r % uR;
      d.w = a.w_down;
      d.blk = ((int64_t)e * (a.H / 16) + ct) * (a.I / 32) + pt * kD;
      const int bs = meta.ent[e][nl];
      d.ho = nl < meta.count[e] ? (((uint32_t)(bs >> 8) * (a.k + 1) + (bs & 0xff)) * a.IM +
                                   pt * kUnit + kq * 8) * 2u
                                : kM8Off;
    }
    return d;
  };
  typename W::Raw dw[kD];
  u32x4 xs[kD];
  auto issue = [&](const Unit& d) {
#pragma unroll
    for (int t = 0; t < kD; ++t) {
      dw[t] = W::load(d.w, d.blk + t, lane);
      xs[t] = __builtin_amdgcn_raw_buffer_load_b128(hrs, d.ho + t * 64u, 0, 0);
    }
  };
  // a wave whose first unit is the shared expert's needs no group list for
  // it: its loads go out before the lists are staged
  const bool early = wave < uS;
  Unit first;
  if (early) {
    first = decode(0);
    issue(first);
  }
  m8_stage(a, meta);
  const int nU = uS + meta.n * uR;
  const int mine = wave < nU ? (nU - 1 - wave) / kWv + 1 : 0;
  // the mix threads' slot weights and row scales, requested now and used at
  // the end
  const int t = threadIdx.x;
  const bool mixer = t < a.B * 16;
  const int b = mixer ? t / 16 : 0, n = t % 16, col = ct * 16 + n;
  float wslot[kM8Slots - 1], sslot[kM8Slots - 1];
#pragma unroll
  for (int s = 0; s < kM8Slots - 1; ++s) {
    const int ss = s < a.k ? s : 0;
    wslot[s] = a.weights[(int64_t)b * a.k + ss];
    if (kFp8) {
      // an id out of range is served as expert 0, as k_moe_group groups it
      const int e = a.idx[(int64_t)b * a.k + ss];
      sslot[s] = a.s_down[(int64_t)((unsigned)e < (unsigned)a.E ? e : 0) * a.H + col];
    } else {
      sslot[s] = 1.f;
    }
  }
  const float s_sh = kFp8 ? a.s_sout[col] : 1.f;
  // unit j's steps, each slot refilled with the next unit's step right after
  // its use (the last unit has none: a separate copy, so no branch sits
  // between a load and its use)
  auto unit = [&](int j, const Unit& nx, auto refill) {
    f32x4_m c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < kD; ++t) {
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(m8_a(xs[t]), W::value(dw[t]), c, 0, 0, 0);
      if (decltype(refill)::value) {
        dw[t] = W::load(nx.w, nx.blk + t, lane);
        xs[t] = __builtin_amdgcn_raw_buffer_load_b128(hrs, nx.ho + t * 64u, 0, 0);
      }
    }
    const int u = wave + j * kWv;
    const bool sh = u < uS;
    const int r = u - uS, e = sh ? 0 : meta.picked[r / uR], pt = sh ? 0 : r % uR;
    const int cnt = sh ? a.B : meta.count[e];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 4 * kq + i;
      if (m >= cnt) continue;
      if (sh) {
        shp[(u * kM8 + m) * 16 + nl] = c[i];
      } else {
        const int bs = meta.ent[e][m];
        part[(((bs >> 8) * (a.k + 1) + (bs & 0xff)) * uR + pt) * 16 + nl] = c[i];
      }
    }
  };
  if (mine > 0) {
    if (!early) {
      first = decode(0);
      issue(first);
    }
    for (int j = 0; j + 1 < mine; ++j) unit(j, decode(j + 1), std::true_type{});
    unit(mine - 1, first, std::false_type{});
  }
  __syncthreads();
  // mix, as k_moe_down's rounding and k_moe_mix: each slot's units in K order,
  // times its row scale, rounded to bf16; the slots in slot order, then the
  // shared expert
  if (!mixer) return;
  float acc = 0.f;
#pragma unroll
  for (int s = 0; s < kM8Slots - 1; ++s) {
    if (s >= a.k) break;
    const float* ps = part + ((b * (a.k + 1) + s) * uR) * 16 + n;
    float raw = ps[0];
    for (int pt = 1; pt < uR; ++pt) raw += ps[pt * 16];
    const float d = rbf(kFp8 ? raw * sslot[s] : raw);
    acc += kF32 ? d * wslot[s] : rbf(d * wslot[s]);
  }
  float sraw = shp[b * 16 + n];
  for (int u = 1; u < uS; ++u) sraw += shp[(u * kM8 + b) * 16 + n];
  const float dsh = rbf(kFp8 ? sraw * s_sh : sraw);
  const int64_t at = (int64_t)b * a.H + col;
  if (kF32) {
    const float y = acc + dsh * (a.w_sscale ? a.sscale[b] : 1.f);
    a.out[at] = a.accumulate ? a.out[at] + y : y;
  } else {
    const float y = rbf(rbf(acc) + dsh);
    if (a.resid)
      a.resid[at] = f2bf(bf2f(a.resid[at]) + rbf(y * a.resid_mult));
    else
      a.out[at] = y;
  }
}

// ---------------------------------------------------------------------------
// An fp8 projection with the HIR's RMSNorm as its prologue, for at most eight
// rows (C5: the input norm + in-projection, the post norm + router, which also
// hands the normalised rows to the experts).  A separate norm launch costs the
// ramp and tail every launch pays (about 4 us); here a block normalises the
// rows itself, into LDS, while its first weight loads are in flight:
//   prologue  wave r normalises row r as tfd_tf_rmsnorm_rows_bf16 does (the
//             same sums in the same order: the same bits) into LDS (block 0
//             also to x_rows)
//   tiles     the block takes a run of `tiles` 16-column tiles; its eight
//             waves split K, read the A operand from LDS and stream the packed
//             fp8 blocks kD steps ahead across tile boundaries; the waves'
//             sums meet in LDS (one buffer, two barriers per tile, so that two
//             blocks fit a compute unit) and one wave in turn applies the scale
//             and the epilogue (bf16 rows, or bf16-valued f32 logits)
// ---------------------------------------------------------------------------
struct Proj8Args {
  const bf16* x;            // [M][ldx] bf16 rows
  int ldx;
  const bf16* gamma;        // [K]
  float eps;
  bf16* x_rows;             // optional [M][ldxr]: the normalised rows
  int ldxr;
  const void* w;            // packed fp8 [N][K] (tfd_pack_skinny_fp8)
  const float* scale;       // [N]
  int M, K, N;
  void* out;                // kEpi 0: bf16 [M][ldo]; 1: f32 [M][ldo]
  int ldo, tiles;
};
constexpr int kP8Waves = 8;
constexpr int kP8Rows = 8;
constexpr int kP8K = 4096;                 // the prologue's chunk map: K = 8 x 512
constexpr int kP8Ld = kP8K + 8;            // LDS row stride (bf16), 16 bytes of pad
// under 80 KB, so that two blocks fit a compute unit
constexpr size_t kP8Lds = (size_t)kP8Rows * kP8Ld * 2 + kP8Waves * kWave * 16;

template <int kEpi, int kD>
__global__ __launch_bounds__(kP8Waves * kWave) void k_proj8_norm(Proj8Args a) {
  using W = M8W<true>;
  extern __shared__ __attribute__((aligned(16))) uint8_t p8_lds[];
  bf16* xs = reinterpret_cast<bf16*>(p8_lds);
  f32x4_m* red = reinterpret_cast<f32x4_m*>(p8_lds + (size_t)kP8Rows * kP8Ld * 2);
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int nl = lane & 15, kq = lane >> 4;
  const int ntiles = (a.N + 15) / 16, ksteps = kP8K / 32;
  constexpr int ns = kP8K / 32 / kP8Waves;        // this wave's steps per tile
  const int t0 = (int)blockIdx.x * a.tiles;
  if (t0 >= ntiles) return;
  const int mine = min(a.tiles, ntiles - t0), total = mine * ns;
  const int k0 = wave * ns;
  typename W::Raw b[kD];
  int jn = 0, sn = 0;
  auto issue = [&](int u) {
    b[u] = W::load(a.w, (int64_t)(t0 + jn) * ksteps + k0 + sn, lane);
    if (++sn == ns && jn + 1 < mine) {
      sn = 0;
      ++jn;
    }
  };
#pragma unroll
  for (int u = 0; u < kD; ++u) issue(u);
  // ---- prologue: the rows' norm into LDS.  Wave r normalises row r exactly
  // as tfd_tf_rmsnorm_rows_bf16 does (rms_norm_x: lane l holds chunks l, l + 64,
  // ..., the squares summed in that order, then the wave's sum), so the rows
  // are that kernel's bit for bit.
  if (wave < a.M) {
    u32x4 xr[kP8K / 512];
    rms_norm_x<kP8K / 512, true>(a.x + (int64_t)wave * a.ldx, a.gamma, kP8K, a.eps, lane, xr);
#pragma unroll
    for (int i = 0; i < kP8K / 512; ++i) {
      const int c = i * kWave + lane;
      *reinterpret_cast<u32x4*>(xs + wave * kP8Ld + c * 8) = xr[i];
      if (a.x_rows && blockIdx.x == 0)
        *reinterpret_cast<u32x4*>(a.x_rows + (int64_t)wave * a.ldxr + c * 8) = xr[i];
    }
  }
  __syncthreads();
  // ---- the tiles
  const bool valid = nl < a.M;
  const bf16* arow = xs + (valid ? nl : 0) * kP8Ld + k0 * 32 + kq * 8;
  f32x4_m c = {0.f, 0.f, 0.f, 0.f};
  int jc = 0, sc = 0;
  auto compute = [&](int u) {
    const u32x4 av = valid ? *reinterpret_cast<const u32x4*>(arow + sc * 32)
                           : u32x4{0u, 0u, 0u, 0u};
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_m, av),
                                                W::value(b[u]), c, 0, 0, 0);
    if (++sc < ns) return;
    const int j = jc++;
    sc = 0;
    red[wave * kWave + lane] = c;
    c = f32x4_m{0.f, 0.f, 0.f, 0.f};
    __syncthreads();
    f32x4_m sum = red[lane];
    const bool mine_ep = wave == (j & (kP8Waves - 1));
    if (mine_ep) {
#pragma unroll
      for (int w = 1; w < kP8Waves; ++w) {
        const f32x4_m v = red[w * kWave + lane];
#pragma unroll
        for (int e = 0; e < 4; ++e) sum[e] += v[e];
      }
    }
    __syncthreads();                               // the sums read: LDS free for the next tile
    const int n = (t0 + j) * 16 + nl;
    if (!mine_ep || n >= a.N) return;
    const float sc_n = a.scale[n];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = 4 * kq + e;
      if (m >= a.M) continue;
      const float y = rbf(sum[e] * sc_n);
      if (kEpi == 0)
        ((bf16*)a.out)[(int64_t)m * a.ldo + n] = f2bf(y);
      else
        ((float*)a.out)[(int64_t)m * a.ldo + n] = y;
    }
  };
  int q0 = 0;
  for (; q0 + kD < total; q0 += kD) {
#pragma unroll
    for (int u = 0; u < kD; ++u) {
      compute(u);
      issue(u);
    }
  }
#pragma unroll
  for (int u = 0; u < kD; ++u) compute(u);
}

// ---------------------------------------------------------------------------
// Gated DeltaNet, one token (torch_ref.py:188-312): one block per (value head,
// sequence).  The block convolves the channels its head reads (its key head's
// q and k, its own v), L2-normalises q and k, updates its [DK][DV] f32 state
// in place and writes the gated, normalised read-out in operand order for the
// out-projection.  A thread owns one value column over half of the key rows.
// ---------------------------------------------------------------------------
struct GdnArgs {
  const float* proj;        // [B][ldp]: conv channels (q | k | v), z, b, a
  int ldp;
  const float* conv_in;     // [B][CONV][KW-1]
  float* conv_out;          // [B][CONV][KW-1] (a different buffer)
  float* state;             // [B][HV][DK][DV]
  const bf16* conv_w;       // [CONV][KW]
  const bf16 *a_log, *dt_bias, *gamma;   // [HV], [HV], [DV]
  bf16* out;                // operand order, 32 x HV*DV
  int hk, hv;
  float l2_eps, rms_eps;
};

template <int kD>
__global__ __launch_bounds__(2 * kD) void k_gdn_step(GdnArgs a) {
  constexpr int kKW = 4;
  const int hv = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int vpk = a.hv / a.hk, hk = hv / vpk;
  const int key = a.hk * kD, val = a.hv * kD, conv = 2 * key + val;
  const float* proj = a.proj + (int64_t)b * a.ldp;
  const float* cin = a.conv_in + (int64_t)b * conv * (kKW - 1);
  float* cout = a.conv_out + (int64_t)b * conv * (kKW - 1);
  __shared__ float q_s[kD], k_s[kD], v_s[kD], red[2][kD], sc[4];
  // this thread's state column slice (thread (dv, half): key rows [half * kD/2,
  // +kD/2)) is requested first, so it streams in while the prologue runs
  const int dv = tid % kD, half = tid / kD;
  constexpr int kRows = kD / 2;
  float* st = a.state + (((int64_t)b * a.hv + hv) * kD + half * kRows) * kD + dv;
  float s[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) s[r] = st[(int64_t)r * kD];
  // ---- conv + SiLU of this head's channels; q/k windows advance once per key head
  {
    const int d = tid % kD;
    const int c = tid < kD ? hk * kD + d : key + hk * kD + d;
    const float m = conv_silu_f32<kD, kKW>(cin + (int64_t)c * (kKW - 1), a.conv_w + (int64_t)c * kKW,
                                           proj[c], cout + (int64_t)c * (kKW - 1), hv % vpk == 0);
    (tid < kD ? q_s : k_s)[d] = m;
    if (tid < kD) {
      const int cv = 2 * key + hv * kD + d;
      v_s[d] = conv_silu_f32<kD, kKW>(cin + (int64_t)cv * (kKW - 1),
                                      a.conv_w + (int64_t)cv * kKW, proj[cv],
                                      cout + (int64_t)cv * (kKW - 1), true);
    }
  }
  __syncthreads();
  // ---- L2 norms of q (threads < kD) and k, beta and g
  {
    const int d = tid % kD;
    const float x = tid < kD ? q_s[d] : k_s[d];
    float ss = wave_sum(x * x);
    if ((tid & (kWave - 1)) == 0) red[0][tid / kWave] = ss;
  }
  __syncthreads();
  if (tid == 0) {
    float sq = 0.f, sk = 0.f;
    for (int w = 0; w < kD / kWave; ++w) sq += red[0][w];
    for (int w = kD / kWave; w < 2 * kD / kWave; ++w) sk += red[0][w];
    sc[0] = rsqrtf(sq + a.l2_eps);
    sc[1] = rsqrtf(sk + a.l2_eps);
    const float braw = proj[conv + val + hv];
    const float araw = proj[conv + val + a.hv + hv];
    sc[2] = sigmoid_f(braw);
    sc[3] = expf(-expf(bf2f(a.a_log[hv])) * softplus_f(araw + bf2f(a.dt_bias[hv])));
  }
  __syncthreads();
  if (tid < kD) {
    q_s[tid] *= sc[0] * rsqrtf((float)kD);          // l2-normalised q times DK^-1/2
    k_s[tid] *= sc[1];
  }
  __syncthreads();
  // ---- the delta rule: thread (dv, half) over key rows [half * kD/2, +kD/2)
  const float decay = sc[3], beta = sc[2];
  float rec = 0.f;
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    s[r] *= decay;
    rec += s[r] * k_s[half * kRows + r];
  }
  red[half][dv] = rec;
  __syncthreads();
  const float delta = (v_s[dv] - (red[0][dv] + red[1][dv])) * beta;
  float rd = 0.f;
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const float u = s[r] + k_s[half * kRows + r] * delta;
    st[(int64_t)r * kD] = u;
    rd += u * q_s[half * kRows + r];
  }
  __syncthreads();                      // red is reused
  red[half][dv] = rd;
  __syncthreads();
  // ---- gated RMS norm over the head's DV values, then out in operand order
  if (tid < kD) {
    const float read = red[0][tid] + red[1][tid];
    float ss = wave_sum(read * read);
    if ((tid & (kWave - 1)) == 0) v_s[tid / kWave] = ss;     // v_s is free now
  }
  __syncthreads();
  if (tid < kD) {
    float ms = 0.f;
    for (int w = 0; w < kD / kWave; ++w) ms += v_s[w];
    ms /= (float)kD;
    const float read = red[0][tid] + red[1][tid];
    const float z = proj[conv + hv * kD + tid];
    const float g = read * rsqrtf(ms + a.rms_eps) * bf2f(a.gamma[tid]) * silu_f(z);
    a.out[xp_off_h(b, hv * kD + tid)] = f2bf(g);
  }
}

// ---------------------------------------------------------------------------
// Mamba2, one token (granite model.py:154-238): one block per (head,
// sequence) for the convolution and the selective-state update (bf16 ops
// rounded as the HIR writes them), then one block per sequence for the gated
// RMS norm over the whole inner width.
// ---------------------------------------------------------------------------
struct MambaArgs {
  const bf16* proj;         // [B][ldp]: gate (EXP) | x B C (CONV) | dt (NH)
  int ldp;
  const bf16* conv_in;      // [B][CONV][KW-1]
  bf16* conv_out;           // [B][CONV][KW-1] (a different buffer)
  float* state;             // [B][NH][PD][NS]
  const bf16 *conv_w, *conv_b;               // [CONV][KW], [CONV]
  const bf16 *a_log, *dt_bias, *d_skip;      // [NH]
  const bf16* gamma;        // [EXP]
  float* gated;             // [B][EXP] work
  float* ssq;               // [B][NH] work
  bf16* out;                // operand order, 32 x EXP
  int nh, ns;               // heads, state width (ngroups 1)
  float eps;
};

__device__ __forceinline__ float conv_silu_bf16(const bf16* cin, const bf16* w, bf16 bias,
                                                float entry, bf16* cout, bool write) {
  constexpr int kKW = 4;
  float win[kKW];
#pragma unroll
  for (int t = 0; t < kKW - 1; ++t) win[t] = bf2f(cin[t]);
  win[kKW - 1] = entry;
  float sum = 0.f;
#pragma unroll
  for (int t = 0; t < kKW; ++t) sum += rbf(win[t] * bf2f(w[t]));   // bf16 window * kernel
  const float pre = rbf(rbf(sum) + bf2f(bias));
  if (write) {
#pragma unroll
    for (int t = 0; t < kKW - 1; ++t) cout[t] = f2bf(win[t + 1]);
  }
  return rbf(silu_f(pre));
}

template <int kPD>
__global__ __launch_bounds__(kBlock) void k_mamba_step(MambaArgs a) {
  constexpr int kKW = 4, kNS = 128;
  constexpr int kLpr = kNS / 4;                   // lanes per state row (4 columns each)
  constexpr int kRpp = kBlock / kLpr;             // rows per pass
  constexpr int kPass = kPD / kRpp;
  const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int exp_ = a.nh * kPD, conv = exp_ + 2 * kNS;
  const bf16* proj = a.proj + (int64_t)b * a.ldp;
  const bf16* cin = a.conv_in + (int64_t)b * conv * (kKW - 1);
  bf16* cout = a.conv_out + (int64_t)b * conv * (kKW - 1);
  __shared__ float x_s[kPD], b_s[kNS], c_s[kNS], dtv[2];
  __shared__ float ss_w[kWavesPerBlock];
  // this thread's four state columns in every pass: 16-byte loads, a row's 32
  // lanes contiguous, all passes' loads issued first (they stream in while the
  // conv and dt prologue runs)
  const int q = tid % kLpr, r0 = tid / kLpr;
  float4* st = reinterpret_cast<float4*>(a.state + ((int64_t)b * a.nh + h) * kPD * kNS) + q;
  float4 sv[kPass];
#pragma unroll
  for (int i = 0; i < kPass; ++i) sv[i] = st[(int64_t)(r0 + kRpp * i) * kLpr];
  for (int i = tid; i < kPD + 2 * kNS; i += kBlock) {
    const int ch = i < kPD ? h * kPD + i : exp_ + (i - kPD);
    const float m = conv_silu_bf16(cin + (int64_t)ch * (kKW - 1), a.conv_w + (int64_t)ch * kKW,
                                   a.conv_b[ch], bf2f(proj[exp_ + ch]),
                                   cout + (int64_t)ch * (kKW - 1), i < kPD || h == 0);
    if (i < kPD)
      x_s[i] = m;
    else if (i < kPD + kNS)
      b_s[i - kPD] = m;
    else
      c_s[i - kPD - kNS] = m;
  }
  if (tid == 0) {
    const float dt = rbf(softplus_f(rbf(bf2f(proj[exp_ + conv + h]) + bf2f(a.dt_bias[h]))));
    dtv[0] = dt;
    dtv[1] = expf(dt * -expf(bf2f(a.a_log[h])));
  }
  __syncthreads();
  const float dt = dtv[0], decay = dtv[1];
  float dtb[4], cq[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    dtb[e] = rbf(dt * b_s[4 * q + e]);
    cq[e] = c_s[4 * q + e];
  }
  const float dsk = bf2f(a.d_skip[h]);
  float g2 = 0.f;
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
    st[(int64_t)p * kLpr] = float4{u[0], u[1], u[2], u[3]};
    rd = group_sum<kLpr>(rd);
    if (q == 0) {
      const float y = rbf(rbf(rd) + rbf(xp * dsk));
      const float gt = y * silu_f(bf2f(proj[h * kPD + p]));
      a.gated[(int64_t)b * exp_ + h * kPD + p] = gt;
      g2 += gt * gt;
    }
  }
  g2 = wave_sum(g2);
  if ((tid & (kWave - 1)) == 0) ss_w[tid / kWave] = g2;
  __syncthreads();
  if (tid == 0) {
    float t = 0.f;
    for (int w = 0; w < kWavesPerBlock; ++w) t += ss_w[w];
    a.ssq[(int64_t)b * a.nh + h] = t;
  }
}

// the gated RMS norm over the whole inner width; grid (chunks of 1024, rows)
__global__ __launch_bounds__(kBlock) void k_mamba_norm(MambaArgs a, int exp_) {
  const int b = blockIdx.y, lane = threadIdx.x & (kWave - 1);
  __shared__ float tot;
  if (threadIdx.x < kWave) {
    float t = 0.f;
    for (int h = lane; h < a.nh; h += kWave) t += a.ssq[(int64_t)b * a.nh + h];
    t = wave_sum(t);
    if (lane == 0) tot = rsqrtf(t / (float)exp_ + a.eps);
  }
  __syncthreads();
  const int i0 = blockIdx.x * kBlock * 4;
  for (int i = i0 + threadIdx.x; i < i0 + kBlock * 4 && i < exp_; i += kBlock)
    a.out[xp_off_h(b, i)] = f2bf(a.gated[(int64_t)b * exp_ + i] * tot * bf2f(a.gamma[i]));
}

// ---------------------------------------------------------------------------
// The f32 residual stream of C4 (torch_ref.py's policy): norms of f32 rows with
// one bf16 rounding of the scaled value (the matmul's cast), residual adds and
// the embedding row lifted to f32.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void k_rmsnorm_f32_rows(const float* __restrict__ x, int ldx,
                                                             const bf16* __restrict__ gamma,
                                                             bf16* out_rows, int ldo,
                                                             bf16* out_packed, int n, float eps) {
  constexpr int kMax4 = 8;                 // n <= 8192: the row stays in registers
  const int b = blockIdx.x, tid = threadIdx.x, n4 = n / 4;
  __shared__ float red[kWavesPerBlock];
  const float4* xr = reinterpret_cast<const float4*>(x + (int64_t)b * ldx);
  float4 v[kMax4];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kMax4; ++i) {
    const int q = tid + kBlock * i;
    v[i] = q < n4 ? xr[q] : float4{0.f, 0.f, 0.f, 0.f};
    ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
  }
  ss = wave_sum(ss);
  if ((tid & (kWave - 1)) == 0) red[tid / kWave] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < kWavesPerBlock; ++w) tot += red[w];
  const float r = rsqrtf(tot / (float)n + eps);
#pragma unroll
  for (int i = 0; i < kMax4; ++i) {
    const int q = tid + kBlock * i;
    if (q < n4) {
      const int c = 4 * q;
      const uint2 g = *reinterpret_cast<const uint2*>(gamma + c);
      const uint2 o = {pack2(v[i].x * r * bf_lo(g.x), v[i].y * r * bf_hi(g.x)),
                       pack2(v[i].z * r * bf_lo(g.y), v[i].w * r * bf_hi(g.y))};
      if (out_rows) *reinterpret_cast<uint2*>(out_rows + (int64_t)b * ldo + c) = o;
      if (out_packed) *reinterpret_cast<uint2*>(out_packed + xp_off_h(b, c)) = o;
    }
  }
}

__global__ __launch_bounds__(kBlock) void k_add_f32_rows(float* __restrict__ acc, int lda,
                                                         const float* __restrict__ add, int ldb,
                                                         int n) {
  const int b = blockIdx.y, i = blockIdx.x * kBlock + threadIdx.x;
  if (i < n) acc[(int64_t)b * lda + i] += add[(int64_t)b * ldb + i];
}

__global__ __launch_bounds__(kBlock) void k_bf16_to_f32_rows(const bf16* __restrict__ src,
                                                             int lds, float* __restrict__ dst,
                                                             int ldd, int n) {
  const int b = blockIdx.y, i = blockIdx.x * kBlock + threadIdx.x;
  if (i < n) dst[(int64_t)b * ldd + i] = bf2f(src[(int64_t)b * lds + i]);
}

// Granite's scaled residual (model.py:502-508, 519-523): out = a + b * m with
// bf16 ops (the product rounded, then the sum); a NULL `a` gives bf16(b * m)
// (the embedding times embedding_multiplier, :615-624).  b is bf16, or f32
// holding bf16 values (the experts' output).
__global__ __launch_bounds__(kBlock) void k_scaled_add_rows(const bf16* __restrict__ a, int lda,
                                                            const void* __restrict__ b, int ldb,
                                                            int b_f32, float m,
                                                            bf16* __restrict__ out, int ldo,
                                                            int n) {
  const int r = blockIdx.y, i = blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  const float bv = b_f32 ? ((const float*)b)[(int64_t)r * ldb + i]
                         : bf2f(((const bf16*)b)[(int64_t)r * ldb + i]);
  const float p = rbf(bv * m);
  out[(int64_t)r * ldo + i] = f2bf(a ? bf2f(a[(int64_t)r * lda + i]) + p : p);
}

}  // namespace

// gate/up + SwiGLU for every group (the registers per lane depend only on the
// hidden size; blocks past a narrower expert's rows leave at once)
template <bool kFp8, bool kF32>
int launch_moe_gateup(const MoeArgs& a, int width, int ny, hipStream_t s) {
  constexpr int kRgu = 1;               // one row per wave: many small blocks, even tails
  const dim3 g1((width + kWavesPerBlock * kRgu - 1) / (kWavesPerBlock * kRgu), ny);
  switch (cmax_for(a.H)) {
    case 1: hipLaunchKernelGGL((k_moe_gateup<kFp8, kF32, 1, kRgu>), g1, dim3(kBlock), 0, s, a); break;
    case 2: hipLaunchKernelGGL((k_moe_gateup<kFp8, kF32, 2, kRgu>), g1, dim3(kBlock), 0, s, a); break;
    case 4: hipLaunchKernelGGL((k_moe_gateup<kFp8, kF32, 4, kRgu>), g1, dim3(kBlock), 0, s, a); break;
    case 8: hipLaunchKernelGGL((k_moe_gateup<kFp8, kF32, 8, kRgu>), g1, dim3(kBlock), 0, s, a); break;
    default: return fail(kUnsupported, "moe_experts: hidden size %d", a.H);
  }
  return 0;
}

// the down projections for the groups kWho selects, whose expert width (K of
// the projection, which sets the chunks a lane holds) is `width`, over `ny`
// groups
template <bool kFp8, int kWho>
int launch_moe_down(const MoeArgs& a, int width, int ny, hipStream_t s) {
  // one pass of four rows per wave: many small blocks with even tails
  // (measured at C5's fp8 shape: two passes no faster)
  constexpr int kPdn = 1;
  constexpr int kRdn = kPdn * (kWave / kDownLanes);
  const dim3 g2((a.H + kWavesPerBlock * kRdn - 1) / (kWavesPerBlock * kRdn), ny);
  // chunks of 8 weights per lane over the 16 lanes of a row
  const int dc = (width / 8 + kDownLanes - 1) / kDownLanes;
  if (dc <= 4)
    hipLaunchKernelGGL((k_moe_down<kFp8, 4, kPdn, kWho>), g2, dim3(kBlock), 0, s, a);
  else if (dc <= 6)
    hipLaunchKernelGGL((k_moe_down<kFp8, 6, kPdn, kWho>), g2, dim3(kBlock), 0, s, a);
  else if (dc <= 8)
    hipLaunchKernelGGL((k_moe_down<kFp8, 8, kPdn, kWho>), g2, dim3(kBlock), 0, s, a);
  else if (dc <= 12)
    hipLaunchKernelGGL((k_moe_down<kFp8, 12, kPdn, kWho>), g2, dim3(kBlock), 0, s, a);
  else if (dc <= 16)
    hipLaunchKernelGGL((k_moe_down<kFp8, 16, kPdn, kWho>), g2, dim3(kBlock), 0, s, a);
  else
    return fail(kUnsupported, "moe_experts: expert width %d", width);
  return 0;
}

// the matrix-core expert pair's limits: a group fits one 16-row tile, a wave's
// share of K in the gate/up (a quarter of the hidden size) is a whole number of
// kM8Depth 32-wide steps, both expert widths are whole numbers of the down's
// units, and the down's unit sums fit its LDS
bool moe8_fits(const MoeArgs& a) {
  return a.B <= kM8 && a.k + 1 <= kM8Slots && a.E <= kMaxExperts &&
         a.H % (32 * kWavesPerBlock * kM8Depth) == 0 && a.I % kM8Unit == 0 &&
         a.IS % kM8Unit == 0 && a.IS / kM8Unit <= kM8SharedUnits &&
         a.B * (a.k + 1) * (a.I / kM8Unit) <= kM8Parts;
}

// route (when asked) and group the entries by expert
void launch_group(const MoeArgs& a, hipStream_t s) {
  if (a.route == TFD_ROUTE_SOFTMAX_TOPK)
    hipLaunchKernelGGL((k_moe_group<0>), dim3(1), dim3(kGroupThreads), 0, s, a);
  else if (a.route == TFD_ROUTE_TOPK_SOFTMAX)
    hipLaunchKernelGGL((k_moe_group<1>), dim3(1), dim3(kGroupThreads), 0, s, a);
  else
    hipLaunchKernelGGL((k_moe_group<-1>), dim3(1), dim3(kGroupThreads), 0, s, a);
}

// packed weights, at most 16 sequences: group, gate/up, down + mix
template <bool kFp8, bool kF32>
int launch_moe8(const MoeArgs& a, hipStream_t s) {
  const int np = a.E < a.B * a.k ? a.E : a.B * a.k;
  const int items = a.IS / 16 + np * (a.I / 16);
  // as many gate/up blocks as are resident at once (one round, no tail)
  static int per_cu[2][2] = {{0, 0}, {0, 0}};
  int& pc = per_cu[kFp8][kF32];
  if (!pc && (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                  &pc, reinterpret_cast<const void*>(&k_moe8_gateup<kFp8, kF32>), kBlock, 0) !=
                  hipSuccess ||
              pc <= 0))
    pc = 2;
  const int cap = pc * compute_units();
  launch_group(a, s);
  hipLaunchKernelGGL((k_moe8_gateup<kFp8, kF32>), dim3(items < cap ? items : cap), dim3(kBlock),
                     0, s, a);
  // whole 768-wide experts as units (C5's width) measured 5% faster than
  // 256-wide units over 16 waves
  if (a.I % 768 == 0 && a.IS % 768 == 0 && a.IS / 768 <= kM8SharedUnits)
    hipLaunchKernelGGL((k_moe8_down<kFp8, kF32, 8, 24>), dim3(a.H / 16), dim3(8 * kWave), 0, s,
                       a);
  else
    hipLaunchKernelGGL((k_moe8_down<kFp8, kF32, 16>), dim3(a.H / 16), dim3(16 * kWave), 0, s, a);
  return launched("moe_experts_packed");
}

template <bool kFp8, bool kF32>
int launch_moe(const MoeArgs& a, hipStream_t s) {
  // picked experts at most min(E, B k), plus the shared one
  const int np = a.E < a.B * a.k ? a.E : a.B * a.k;
  const dim3 g3((a.H + kBlock - 1) / kBlock, a.B);
  launch_group(a, s);
  // gate/up in one launch; the down projections in one launch when the shared
  // expert is as wide as the routed ones, else one for each width (a lane's
  // chunk registers are sized by the width)
  int rc = launch_moe_gateup<kFp8, kF32>(a, a.I > a.IS ? a.I : a.IS, np + 1, s);
  if (rc) return rc;
  if (a.I == a.IS)
    rc = launch_moe_down<kFp8, 0>(a, a.I, np + 1, s);
  else if ((rc = launch_moe_down<kFp8, 1>(a, a.I, np, s)) == 0)
    rc = launch_moe_down<kFp8, 2>(a, a.IS, 1, s);
  if (rc) return rc;
  hipLaunchKernelGGL((k_moe_mix<kF32>), g3, dim3(kBlock), 0, s, a);
  return launched("moe_experts");
}

extern "C" {

int tfd_route_topk(const float* logits, int ldl, int rows, int experts, int k, int mode,
                   float* weights, int32_t* idx, void* stream) {
  if (!logits || !weights || !idx) return fail(kBadArg, "route_topk: null pointer");
  if (rows <= 0 || experts <= 0 || experts > 256 || k <= 0 || k > experts || k > kWave ||
      ldl < experts || (mode != TFD_ROUTE_SOFTMAX_TOPK && mode != TFD_ROUTE_TOPK_SOFTMAX))
    return fail(kBadShape, "route_topk: rows=%d experts=%d (<= 256) k=%d mode=%d", rows,
                experts, k, mode);
  auto s = (hipStream_t)stream;
  if (mode == TFD_ROUTE_SOFTMAX_TOPK)
    hipLaunchKernelGGL(k_route<0>, dim3(rows), dim3(kWave), 0, s, logits, ldl, experts, k,
                       weights, (int*)idx);
  else
    hipLaunchKernelGGL(k_route<1>, dim3(rows), dim3(kWave), 0, s, logits, ldl, experts, k,
                       weights, (int*)idx);
  return launched("route_topk");
}

}  // extern "C"

namespace {

// the checks and the device-side arguments shared by the two expert entries
// (the packed one keeps no partials)
int moe_args(const TfdMoeArgs* args, bool partials, const char* who, MoeArgs& a) {
  if (!args) return fail(kBadArg, "%s: null args", who);
  const TfdMoeArgs& t = *args;
  if (!t.x || !t.weights || !t.idx || !t.w_gate || !t.w_up || !t.w_down || !t.w_shared_in ||
      !t.w_shared_out || !t.hidden || (partials && !t.partial) || !t.groups || (!t.out && !t.resid) ||
      (t.fp8 && (!t.s_gate || !t.s_up || !t.s_down || !t.s_shared_in || !t.s_shared_out)) ||
      (t.w_shared_scale && (!t.shared_scale || t.fp8)))
    return fail(kBadArg, "%s: null pointer or a shared-expert gate with fp8 weights", who);
  if (t.rows <= 0 || t.rows > 65535 || t.k <= 0 || t.k > 64 || t.experts <= 0 ||
      t.experts > kMaxExperts || t.hidden_size % 64 || t.hidden_size > 4096 || t.inter % 64 ||
      t.inter > 2048 || t.shared_inter % 64 || t.shared_inter > 2048 ||
      t.hidden_ld < t.inter || t.hidden_ld < t.shared_inter || t.hidden_ld % 8)
    return fail(kBadShape, "%s: rows=%d k=%d experts=%d (<= 256) H=%d (<= 4096) "
                "I=%d IS=%d (<= 2048) ld=%d", who, t.rows, t.k, t.experts, t.hidden_size, t.inter,
                t.shared_inter, t.hidden_ld);
  a.x = (const bf16*)t.x;
  a.weights = t.weights;
  a.idx = (const int*)t.idx;
  a.w_gate = t.w_gate;
  a.w_up = t.w_up;
  a.w_down = t.w_down;
  a.s_gate = t.s_gate;
  a.s_up = t.s_up;
  a.s_down = t.s_down;
  a.w_sin = t.w_shared_in;
  a.w_sout = t.w_shared_out;
  a.s_sin = t.s_shared_in;
  a.s_sout = t.s_shared_out;
  a.w_sscale = (const bf16*)t.w_shared_scale;
  a.hidden = (bf16*)t.hidden;
  a.sscale = t.shared_scale;
  a.partial = t.partial;
  a.groups = (int*)t.groups;
  a.out = t.out;
  a.B = t.rows;
  a.H = t.hidden_size;
  a.I = t.inter;
  a.IS = t.shared_inter;
  a.IM = t.hidden_ld;
  a.k = t.k;
  a.E = t.experts;
  a.accumulate = t.accumulate;
  a.resid = (bf16*)t.resid;
  a.resid_mult = t.resid_mult;
  a.logits = t.logits;
  a.ldl = t.ldl;
  a.route = t.route == TFD_MOE_ROUTE_SOFTMAX_TOPK   ? TFD_ROUTE_SOFTMAX_TOPK
            : t.route == TFD_MOE_ROUTE_TOPK_SOFTMAX ? TFD_ROUTE_TOPK_SOFTMAX
                                                    : -1;
  a.err = t.err;
  if (t.route < TFD_MOE_ROUTE_GIVEN || t.route > TFD_MOE_ROUTE_TOPK_SOFTMAX ||
      (t.route != TFD_MOE_ROUTE_GIVEN && (!t.logits || t.ldl < t.experts || t.k > kWave)))
    return fail(kBadArg, "%s: route %d (0..2) needs logits with ldl >= experts and "
                "k <= 64", who, t.route);
  if (t.accumulate && t.policy != TFD_POLICY_F32)
    return fail(kUnsupported, "%s: accumulate needs the f32 policy", who);
  if (t.resid && t.policy != TFD_POLICY_BF16)
    return fail(kUnsupported, "%s: resid needs the bf16 policy", who);
  if (t.policy != TFD_POLICY_F32 && t.policy != TFD_POLICY_BF16)
    return fail(kBadArg, "%s: policy %d", who, t.policy);
  if (t.fp8 && t.policy != TFD_POLICY_BF16)
    return fail(kUnsupported, "%s: fp8 weights with the f32 policy are not built", who);
  return 0;
}

}  // namespace

extern "C" {

int tfd_moe_experts(const TfdMoeArgs* args, void* stream) {
  MoeArgs a;
  if (int rc = moe_args(args, true, "moe_experts", a)) return rc;
  auto s = (hipStream_t)stream;
  if (args->fp8) return launch_moe<true, false>(a, s);
  if (args->policy == TFD_POLICY_F32) return launch_moe<false, true>(a, s);
  return launch_moe<false, false>(a, s);
}

int tfd_proj8_norm(const TfdProj8NormArgs* args, void* stream) {
  if (!args) return fail(kBadArg, "proj8_norm: null args");
  const TfdProj8NormArgs& t = *args;
  if (!t.x || !t.gamma || !t.w || !t.scale || !t.out)
    return fail(kBadArg, "proj8_norm: null pointer");
  if (t.rows <= 0 || t.rows > kP8Rows || t.K != kP8K || t.N <= 0 || t.ldx < t.K ||
      t.ldo < t.N || (t.x_rows && t.ldxr < t.K) ||
      (t.epilogue != TFD_EPI_STORE && t.epilogue != TFD_EPI_LOGITS))
    return fail(kBadShape, "proj8_norm: rows=%d (1..%d) K=%d (%d) N=%d ldx=%d ldo=%d "
                "epilogue=%d (store or logits)", t.rows, kP8Rows, t.K, kP8K, t.N, t.ldx, t.ldo,
                t.epilogue);
  Proj8Args a;
  a.x = (const bf16*)t.x;
  a.ldx = t.ldx;
  a.gamma = (const bf16*)t.gamma;
  a.eps = t.eps;
  a.x_rows = (bf16*)t.x_rows;
  a.ldxr = t.ldxr;
  a.w = t.w;
  a.scale = t.scale;
  a.M = t.rows;
  a.K = t.K;
  a.N = t.N;
  a.out = t.out;
  a.ldo = t.ldo;
  const int ntiles = (t.N + 15) / 16;
  const void* k = t.epilogue == TFD_EPI_STORE
                      ? reinterpret_cast<const void*>(&k_proj8_norm<0, 16>)
                      : reinterpret_cast<const void*>(&k_proj8_norm<1, 16>);
  // as many blocks as are resident at once, each the same number of tiles (the
  // LDS attribute and the occupancy are set per device)
  static int per_cu[64][2] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return fail(kUnsupported, "proj8_norm: device %d", dev);
  int& pc = per_cu[dev][t.epilogue == TFD_EPI_STORE ? 0 : 1];
  if (!pc) {
    if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kP8Lds) !=
        hipSuccess)
      return fail(kUnsupported, "proj8_norm: %d bytes of LDS refused", (int)kP8Lds);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&pc, k, kP8Waves * kWave, kP8Lds) !=
            hipSuccess || pc <= 0)
      pc = 1;
  }
  const int cap = pc * compute_units();
  a.tiles = (ntiles + cap - 1) / cap;
  const dim3 grid((ntiles + a.tiles - 1) / a.tiles);
  auto s = (hipStream_t)stream;
  if (t.epilogue == TFD_EPI_STORE)
    hipLaunchKernelGGL((k_proj8_norm<0, 16>), grid, dim3(kP8Waves * kWave), kP8Lds, s, a);
  else
    hipLaunchKernelGGL((k_proj8_norm<1, 16>), grid, dim3(kP8Waves * kWave), kP8Lds, s, a);
  return launched("proj8_norm");
}

int tfd_moe_experts_packed(const TfdMoeArgs* args, void* stream) {
  MoeArgs a;
  if (int rc = moe_args(args, false, "moe_experts_packed", a)) return rc;
  if (!moe8_fits(a))
    return fail(kBadShape, "moe_experts_packed: rows=%d (<= 16) k=%d (<= 16) H=%d (a multiple "
                "of 1024) I=%d IS=%d (multiples of 256, IS <= 2048, rows (k + 1) I / 256 <= 1024)",
                a.B, a.k, a.H, a.I, a.IS);
  auto s = (hipStream_t)stream;
  if (args->fp8) return launch_moe8<true, false>(a, s);
  if (args->policy == TFD_POLICY_F32) return launch_moe8<false, true>(a, s);
  return launch_moe8<false, false>(a, s);
}

int tfd_gdn_step(const TfdGdnArgs* args, void* stream) {
  if (!args) return fail(kBadArg, "gdn_step: null args");
  const TfdGdnArgs& t = *args;
  if (!t.proj || !t.conv_in || !t.conv_out || !t.state || !t.conv_w || !t.a_log ||
      !t.dt_bias || !t.gamma || !t.out || t.conv_in == t.conv_out)
    return fail(kBadArg, "gdn_step: null pointer, or conv_out == conv_in");
  if (t.rows <= 0 || t.rows > kMaxRowsH || t.head_k_dim != 128 || t.head_v_dim != 128 ||
      t.key_heads <= 0 || t.value_heads % t.key_heads || t.conv_kernel != 4 ||
      t.proj_ld < 2 * t.key_heads * 128 + 2 * t.value_heads * 128 + 2 * t.value_heads)
    return fail(kBadShape, "gdn_step: rows=%d (1..32) dk=%d dv=%d (128) hk=%d hv=%d kw=%d",
                t.rows, t.head_k_dim, t.head_v_dim, t.key_heads, t.value_heads,
                t.conv_kernel);
  GdnArgs a;
  a.proj = t.proj;
  a.ldp = t.proj_ld;
  a.conv_in = t.conv_in;
  a.conv_out = t.conv_out;
  a.state = t.state;
  a.conv_w = (const bf16*)t.conv_w;
  a.a_log = (const bf16*)t.a_log;
  a.dt_bias = (const bf16*)t.dt_bias;
  a.gamma = (const bf16*)t.gamma;
  a.out = (bf16*)t.out;
  a.hk = t.key_heads;
  a.hv = t.value_heads;
  a.l2_eps = t.l2_eps;
  a.rms_eps = t.rms_eps;
  hipLaunchKernelGGL(k_gdn_step<128>, dim3(t.value_heads, t.rows), dim3(256), 0,
                     (hipStream_t)stream, a);
  return launched("gdn_step");
}

int tfd_mamba_step(const TfdMambaArgs* args, void* stream) {
  if (!args) return fail(kBadArg, "mamba_step: null args");
  const TfdMambaArgs& t = *args;
  if (!t.proj || !t.conv_in || !t.conv_out || !t.state || !t.conv_w || !t.conv_b ||
      !t.a_log || !t.dt_bias || !t.d_skip || !t.gamma || !t.gated || !t.ssq || !t.out ||
      t.conv_in == t.conv_out)
    return fail(kBadArg, "mamba_step: null pointer, or conv_out == conv_in");
  if (t.rows <= 0 || t.rows > kMaxRowsH || t.head_dim != 64 || t.state_dim != 128 ||
      t.groups != 1 || t.conv_kernel != 4 || t.heads <= 0 ||
      t.proj_ld < 2 * t.heads * 64 + 2 * 128 + t.heads)
    return fail(kBadShape, "mamba_step: rows=%d (1..32) heads=%d hd=%d (64) ns=%d (128) "
                "groups=%d (1) kw=%d (4)", t.rows, t.heads, t.head_dim, t.state_dim, t.groups,
                t.conv_kernel);
  MambaArgs a;
  a.proj = (const bf16*)t.proj;
  a.ldp = t.proj_ld;
  a.conv_in = (const bf16*)t.conv_in;
  a.conv_out = (bf16*)t.conv_out;
  a.state = t.state;
  a.conv_w = (const bf16*)t.conv_w;
  a.conv_b = (const bf16*)t.conv_b;
  a.a_log = (const bf16*)t.a_log;
  a.dt_bias = (const bf16*)t.dt_bias;
  a.d_skip = (const bf16*)t.d_skip;
  a.gamma = (const bf16*)t.gamma;
  a.gated = t.gated;
  a.ssq = t.ssq;
  a.out = (bf16*)t.out;
  a.nh = t.heads;
  a.ns = 128;
  a.eps = t.eps;
  auto s = (hipStream_t)stream;
  hipLaunchKernelGGL(k_mamba_step<64>, dim3(t.heads, t.rows), dim3(kBlock), 0, s, a);
  hipLaunchKernelGGL(k_mamba_norm, dim3((t.heads * 64 + 4 * kBlock - 1) / (4 * kBlock), t.rows),
                     dim3(kBlock), 0, s, a, t.heads * 64);
  return launched("mamba_step");
}

int tfd_rmsnorm_f32_rows(const float* x, int ldx, const void* gamma, void* out_rows, int ldo,
                         void* out_packed, int rows, int n, float eps, void* stream) {
  if (!x || !gamma || (!out_rows && !out_packed)) return fail(kBadArg, "rmsnorm_f32: null pointer");
  if (rows <= 0 || n <= 0 || n > 8192 || n % 4 || ldx < n || ldx % 4 ||
      (out_rows && (ldo < n || ldo % 4)) || (out_packed && (rows > kMaxRowsH || n % 32)))
    return fail(kBadShape, "rmsnorm_f32: rows=%d n=%d (a multiple of 4, <= 8192) ldx=%d ldo=%d",
                rows, n, ldx, ldo);
  hipLaunchKernelGGL(k_rmsnorm_f32_rows, dim3(rows), dim3(kBlock), 0, (hipStream_t)stream, x, ldx,
                     (const bf16*)gamma, (bf16*)out_rows, ldo, (bf16*)out_packed, n, eps);
  return launched("rmsnorm_f32_rows");
}

int tfd_add_f32_rows(float* acc, int lda, const float* add, int ldb, int rows, int n,
                     void* stream) {
  if (!acc || !add) return fail(kBadArg, "add_f32: null pointer");
  if (rows <= 0 || n <= 0 || lda < n || ldb < n)
    return fail(kBadShape, "add_f32: rows=%d n=%d", rows, n);
  hipLaunchKernelGGL(k_add_f32_rows, dim3((n + kBlock - 1) / kBlock, rows), dim3(kBlock), 0,
                     (hipStream_t)stream, acc, lda, add, ldb, n);
  return launched("add_f32_rows");
}

int tfd_bf16_to_f32_rows(const void* src, int lds, float* dst, int ldd, int rows, int n,
                         void* stream) {
  if (!src || !dst) return fail(kBadArg, "bf16_to_f32: null pointer");
  if (rows <= 0 || n <= 0 || lds < n || ldd < n)
    return fail(kBadShape, "bf16_to_f32: rows=%d n=%d", rows, n);
  hipLaunchKernelGGL(k_bf16_to_f32_rows, dim3((n + kBlock - 1) / kBlock, rows), dim3(kBlock), 0,
                     (hipStream_t)stream, (const bf16*)src, lds, dst, ldd, n);
  return launched("bf16_to_f32_rows");
}

int tfd_scaled_add_rows(const void* a, int lda, const void* b, int ldb, int b_f32, float m,
                        void* out, int ldo, int rows, int n, void* stream) {
  if (!b || !out) return fail(kBadArg, "scaled_add: null pointer");
  if (rows <= 0 || n <= 0 || (a && lda < n) || ldb < n || ldo < n)
    return fail(kBadShape, "scaled_add: rows=%d n=%d", rows, n);
  hipLaunchKernelGGL(k_scaled_add_rows, dim3((n + kBlock - 1) / kBlock, rows), dim3(kBlock), 0,
                     (hipStream_t)stream, (const bf16*)a, lda, b, ldb, b_f32, m, (bf16*)out, ldo,
                     n);
  return launched("scaled_add_rows");
}

}  // extern "C"

