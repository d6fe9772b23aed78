// GQA decode attention of the hybrid models' full-attention layers, for gfx950.
//
//  * Qwen3.5 (workload C4): 256-wide heads, 8 query heads per kv head, per-head
//    RMSNorm of q and k, rotate-half RoPE on the leading `rot` dims, sigmoid
//    output gate; f32 arithmetic (the example's plain-torch twin).
//  * Granite-4.0-H (workload C5): 128-wide heads, 4 query heads per kv head, no
//    position embedding; bf16 ops rounded as the HIR writes them (products and
//    sums), the softmax in f32.
//
// The KV cache is the dense path's paged layout ([pages][kv_heads][16][head_dim]
// bf16).  Two launches per layer, both over (split, kv head, sequence):
//   scores  the block whose split holds this token's position appends its K/V
//           to the cache; every block scores its split for the kv head's query
//           heads and records each head's split maximum m and sum of exp(x - m);
//   pv      M = max m, S = sum l exp(m - M) over the splits (in split order),
//           p = exp(x - M) / S (C5: rounded to bf16), split partials of
//           sum p v; the last split of a (sequence, kv head) to finish adds the
//           partials in split order and writes o_proj's input in operand order.
// The softmax's sum is thus taken per split and rescaled, where the reference
// sums exp(x - M) in one pass: the two differ by f32 rounding only.

#include "decode_phases.h"
#include "host_common.h"
#include "tf_hybrid.h"

using namespace tfd;
using namespace tfd_host;

namespace {

constexpr int kMaxSplitLen = 512;
constexpr int kMaxRowsG = 32;

struct GqaArgs {
  const void* qkv;
  int ldq;
  const bf16 *gamma_q, *gamma_k, *cos_t, *sin_t;
  int rope_rows, rot;
  const int* pos;
  const int* table;
  int max_pages;
  bf16 *kpool, *vpool;
  int num_pages;
  int hq, hkv;
  float scale, eps;
  float* scores;
  int sstride;
  float* stats;   // [B][HQ][nsplit][2]: split max, split sum of exp(x - max)
  float* part;    // [B][HQ][nsplit][D]
  int* counters;  // [B][HKV]
  int nsplit, split_len;
  bf16* out;      // operand order, 32 x HQ * D
  int* err;
};

__device__ __forceinline__ int64_t xp_off_g(int m, int k) {
  return ((int64_t)((k >> 5) * 2 + (m >> 4)) * 64 + (m & 15) + 16 * ((k >> 3) & 3)) * 8 +
         (k & 7);
}

__device__ __forceinline__ void unpack8(const u32x4 w, float (&v)[8]) {
  v[0] = bf_lo(w.x); v[1] = bf_hi(w.x); v[2] = bf_lo(w.y); v[3] = bf_hi(w.y);
  v[4] = bf_lo(w.z); v[5] = bf_hi(w.z); v[6] = bf_lo(w.w); v[7] = bf_hi(w.w);
}

// position P lies inside the page table (and, with RoPE, the rope table)
__device__ __forceinline__ bool pos_ok(const GqaArgs& a, int P, bool rope) {
  return P >= 0 && P < a.max_pages * kPage && (!rope || P < a.rope_rows);
}

// cache row of position j of (sequence b, kv head h), or -1 for a bad page
template <int kD>
__device__ __forceinline__ int64_t cache_row(const GqaArgs& a, int b, int j, int h) {
  const int page = a.table[(int64_t)b * a.max_pages + j / kPage];
  if (page < 0 || page >= a.num_pages) return -1;
  return page_row(page, j, a.hkv, h, kD);
}

// The split's page ids, staged in LDS once so that no cache load waits on a
// page-table load; a bad entry raises kErrPageRange and reads page 0 instead.
constexpr int kMaxSplitPages = kMaxSplitLen / kPage;
__device__ __forceinline__ void stage_pages(const GqaArgs& a, int b, int j0, int n,
                                            int (&pg_s)[kMaxSplitPages]) {
  const int npg = (n + kPage - 1) / kPage;
  if ((int)threadIdx.x < npg) {
    int page = a.table[(int64_t)b * a.max_pages + j0 / kPage + threadIdx.x];
    if (page < 0 || page >= a.num_pages) {
      raise_error(a.err, kErrPageRange);
      page = 0;
    }
    pg_s[threadIdx.x] = page;
  }
}

// Positions per split: split_len when positive; when 0, derived from the
// sequence's position so that its context spreads evenly over the nsplit
// splits -- ceil((P + 1) / nsplit) rounded up to a page, at least kMinSplitLen
// (the host guarantees nsplit * kMaxSplitLen covers the cache, so it never
// exceeds kMaxSplitLen).  Both launches of a layer read the same position.
constexpr int kMinSplitLen = 64;
__device__ __forceinline__ int split_len_of(const GqaArgs& a, int P) {
  if (a.split_len > 0) return a.split_len;
  int n = (P + a.nsplit) / a.nsplit;                  // ceil((P + 1) / nsplit)
  n = (n + kPage - 1) / kPage * kPage;
  n = n > kMinSplitLen ? n : kMinSplitLen;
  return n < kMaxSplitLen ? n : kMaxSplitLen;
}

// Positions are walked kU passes at a time: every load of the batch is issued
// before the first is used (positions past the split re-read its last row).
constexpr int kU = 4;

// ---------------------------------------------------------------------------
// scores
// ---------------------------------------------------------------------------
template <int kD, int kG, bool kF32>
__global__ __launch_bounds__(kBlock) void k_gqa_scores(GqaArgs a) {
  constexpr int kLpp = kD / 8;          // lanes per cached position (8 dims each)
  constexpr int kPpi = kBlock / kLpp;   // positions per pass of the block
  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int lane = tid & (kWave - 1), wave = tid / kWave;
  __shared__ float qk_s[kG + 1][kD];    // the query heads, then this token's key
  __shared__ float sc[kG][kMaxSplitLen];
  __shared__ int pg_s[kMaxSplitPages];
  const int P = a.pos[b];
  if (!pos_ok(a, P, kF32)) {
    if (split == 0 && kvh == 0 && tid == 0) raise_error(a.err, kErrPosRange);
    return;
  }
  const int slen = split_len_of(a, P);
  const int j0 = split * slen;
  if (j0 > P) return;
  const int j1 = min(j0 + slen, P + 1), n = j1 - j0;
  const bool owner = P < j1;            // this split appends the token's K/V
  const int nrows = kG + (owner ? 1 : 0);
  // ---- this token's query heads (and key head): C4 normalises them per head
  for (int r = wave; r < nrows; r += kWavesPerBlock) {
    const int64_t off = (int64_t)b * a.ldq +
                        (r < kG ? (int64_t)(kvh * kG + r) * (kF32 ? 2 * kD : kD)
                                : (int64_t)a.hq * (kF32 ? 2 * kD : kD) + (int64_t)kvh * kD);
    constexpr int kPer = kD / kWave;
    float x[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int d = lane + kWave * i;
      x[i] = kF32 ? ((const float*)a.qkv)[off + d] : bf2f(((const bf16*)a.qkv)[off + d]);
    }
    if (kF32) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < kPer; ++i) ss += x[i] * x[i];
      ss = wave_sum(ss);
      const float rs = rsqrtf(ss / (float)kD + a.eps);
      const bf16* gm = r < kG ? a.gamma_q : a.gamma_k;
#pragma unroll
      for (int i = 0; i < kPer; ++i) x[i] = x[i] * rs * bf2f(gm[lane + kWave * i]);
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) qk_s[r][lane + kWave * i] = x[i];
  }
  stage_pages(a, b, j0, n, pg_s);
  __syncthreads();
  if (kF32) {
    // rotate-half RoPE on the leading rot dims: x*cos + rotate_half(x)*sin
    constexpr int kMaxPer = ((kG + 1) * kD + kBlock - 1) / kBlock;
    const int h2 = a.rot / 2, tot = nrows * a.rot;
    const bf16* cs = a.cos_t + (int64_t)P * a.rot;
    const bf16* sn = a.sin_t + (int64_t)P * a.rot;
    float t[kMaxPer];
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k) {
      const int idx = tid + k * kBlock;
      if (idx < tot) {
        const int r = idx / a.rot, i = idx % a.rot;
        const float v = qk_s[r][i];
        const float partner = i < h2 ? -qk_s[r][i + h2] : qk_s[r][i - h2];
        t[k] = v * bf2f(cs[i]) + partner * bf2f(sn[i]);
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k) {
      const int idx = tid + k * kBlock;
      if (idx < tot) qk_s[idx / a.rot][idx % a.rot] = t[k];
    }
    __syncthreads();
    for (int idx = tid; idx < kG * kD; idx += kBlock) qk_s[idx / kD][idx % kD] *= a.scale;
    __syncthreads();
  }
  // ---- append this token's key and value
  if (owner && tid < kD) {
    const int64_t row = cache_row<kD>(a, b, P, kvh);
    if (row < 0) {
      raise_error(a.err, kErrPageRange);
    } else {
      const int64_t voff = (int64_t)b * a.ldq + (int64_t)a.hq * (kF32 ? 2 * kD : kD) +
                           (int64_t)(a.hkv + kvh) * kD + tid;
      a.kpool[row + tid] = f2bf(qk_s[kG][tid]);
      a.vpool[row + tid] = kF32 ? f2bf(((const float*)a.qkv)[voff]) : ((const bf16*)a.qkv)[voff];
    }
  }
  // ---- scores of the split: kLpp lanes per position, the query in registers
  const int li = tid % kLpp, pg = tid / kLpp;
  float qr[kG][8];
#pragma unroll
  for (int g = 0; g < kG; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) qr[g][e] = qk_s[g][li * 8 + e];
  float* srow = a.scores + ((int64_t)b * a.hq + kvh * kG) * a.sstride;
  for (int jb = 0; jb < n; jb += kPpi * kU) {
    u32x4 kw[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int jj = min(jb + u * kPpi + pg, n - 1);
      kw[u] = load16(a.kpool + page_row(pg_s[jj / kPage], j0 + jj, a.hkv, kvh, kD) + li * 8);
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int jj = jb + u * kPpi + pg;
      float kv[8];
      if (j0 + jj == P) {
#pragma unroll
        for (int e = 0; e < 8; ++e) kv[e] = qk_s[kG][li * 8 + e];
      } else {
        unpack8(kw[u], kv);
      }
      float acc[kG];
#pragma unroll
      for (int g = 0; g < kG; ++g) {
        acc[g] = 0.f;
        if constexpr (kF32) {
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[g] += qr[g][e] * kv[e];
        } else {
          // each product rounded to bf16, two at a time by one convert, and
          // both added by one bf16 dot against (1, 1)
#pragma unroll
          for (int e = 0; e < 8; e += 2)
            acc[g] = add_rounded2(acc[g], qr[g][e] * kv[e], qr[g][e + 1] * kv[e + 1]);
        }
        acc[g] = group_sum<kLpp>(acc[g]);
      }
      if (li == 0 && jj < n) {
#pragma unroll
        for (int g = 0; g < kG; ++g) {
          const float sv = kF32 ? acc[g] : rbf(acc[g]) * a.scale;
          sc[g][jj] = sv;
          srow[(int64_t)g * a.sstride + j0 + jj] = sv;
        }
      }
    }
  }
  __syncthreads();
  // ---- the split's maximum and sum of exp(x - max), per query head
  for (int g = wave; g < kG; g += kWavesPerBlock) {
    float m = kNegInf;
    for (int jj = lane; jj < n; jj += kWave) m = fmaxf(m, sc[g][jj]);
    m = wave_max(m);
    float l = 0.f;
    for (int jj = lane; jj < n; jj += kWave) l += expf(sc[g][jj] - m);
    l = wave_sum(l);
    if (lane == 0) {
      float* st = a.stats + (((int64_t)b * a.hq + kvh * kG + g) * a.nsplit + split) * 2;
      st[0] = m;
      st[1] = l;
    }
  }
}

// ---------------------------------------------------------------------------
// probabilities, P.V partials and the last split's merge
// ---------------------------------------------------------------------------
template <int kD, int kG, bool kF32>
__global__ __launch_bounds__(kBlock) void k_gqa_pv(GqaArgs a) {
  constexpr int kLpp = kD / 8, kPpi = kBlock / kLpp;
  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int lane = tid & (kWave - 1), wave = tid / kWave;
  __shared__ float Ms[kG], Ss[kG];
  __shared__ float p_s[kG][kMaxSplitLen];
  __shared__ float red[kWavesPerBlock][kG][kD];
  __shared__ int pg_s[kMaxSplitPages];
  __shared__ int is_last;
  const int P = a.pos[b];
  if (!pos_ok(a, P, kF32)) return;      // raised by the scores launch
  const int slen = split_len_of(a, P);
  const int nlive = P / slen + 1;
  if (split >= nlive) return;
  const int j0 = split * slen, j1 = min(j0 + slen, P + 1), n = j1 - j0;
  const int hq0 = kvh * kG;
  if (tid < kG) {
    const float* st = a.stats + ((int64_t)b * a.hq + hq0 + tid) * a.nsplit * 2;
    float M = kNegInf;
    for (int s = 0; s < nlive; ++s) M = fmaxf(M, st[2 * s]);
    float S = 0.f;
    for (int s = 0; s < nlive; ++s) S += st[2 * s + 1] * expf(st[2 * s] - M);
    Ms[tid] = M;
    Ss[tid] = S;
  }
  stage_pages(a, b, j0, n, pg_s);
  __syncthreads();
  const float* srow = a.scores + ((int64_t)b * a.hq + hq0) * a.sstride;
  for (int i = tid; i < kG * n; i += kBlock) {
    const int g = i / n, jj = i % n;
    const float p = expf(srow[(int64_t)g * a.sstride + j0 + jj] - Ms[g]) / Ss[g];
    p_s[g][jj] = kF32 ? p : rbf(p);
  }
  __syncthreads();
  const int li = tid % kLpp, pg = tid / kLpp;
  float acc[kG][8];
#pragma unroll
  for (int g = 0; g < kG; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  for (int jb = 0; jb < n; jb += kPpi * kU) {
    u32x4 vw[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int jj = min(jb + u * kPpi + pg, n - 1);
      vw[u] = load16(a.vpool + page_row(pg_s[jj / kPage], j0 + jj, a.hkv, kvh, kD) + li * 8);
    }
    if constexpr (kF32) {
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int jj = jb + u * kPpi + pg;
        if (jj < n) {
          float v[8];
          unpack8(vw[u], v);
#pragma unroll
          for (int g = 0; g < kG; ++g) {
            const float p = p_s[g][jj];
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[g][e] += p * v[e];
          }
        }
      }
    } else {
      // positions u and u + 1 in pairs: their rounded products p * v meet in
      // one convert and one bf16 dot; a position past the split has p = 0
      // (its row, a re-read of the split's last, is finite)
      static_assert(kU % 2 == 0, "positions pair up");
#pragma unroll
      for (int u = 0; u < kU; u += 2) {
        const int ja = jb + u * kPpi + pg, jb2 = ja + kPpi;
        float va[8], vb[8];
        unpack8(vw[u], va);
        unpack8(vw[u + 1], vb);
#pragma unroll
        for (int g = 0; g < kG; ++g) {
          const float pa = ja < n ? p_s[g][ja] : 0.f;
          const float pb = jb2 < n ? p_s[g][jb2] : 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[g][e] = add_rounded2(acc[g][e], pa * va[e], pb * vb[e]);
        }
      }
    }
  }
  // positions of a wave sit kLpp lanes apart; then the waves, in order
#pragma unroll
  for (int m = kLpp; m < kWave; m <<= 1)
#pragma unroll
    for (int g = 0; g < kG; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] += __shfl_xor(acc[g][e], m, kWave);
  if (lane < kLpp) {
#pragma unroll
    for (int g = 0; g < kG; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) red[wave][g][li * 8 + e] = acc[g][e];
  }
  __syncthreads();
  for (int o = tid; o < kG * kD; o += kBlock) {
    const int g = o / kD, d = o % kD;
    float s = red[0][g][d];
#pragma unroll
    for (int w = 1; w < kWavesPerBlock; ++w) s += red[w][g][d];
    coh_stf(&a.part[(((int64_t)b * a.hq + hq0 + g) * a.nsplit + split) * kD + d], s);
  }
  stores_done();
  __syncthreads();
  if (tid == 0) {
    const int ticket = atomicAdd(&a.counters[b * a.hkv + kvh], 1);
    is_last = ticket == nlive - 1;
  }
  __syncthreads();
  if (!is_last) return;
  // four outputs per thread and pass; the splits' partials arrive in batches of
  // kBatch independent 16-byte device-coherent loads, added in split order
  constexpr int kBatch = 8;
  for (int o4 = tid; o4 < kG * kD / 4; o4 += kBlock) {
    const int g = (o4 * 4) / kD, d = (o4 * 4) % kD;
    const uint32_t base =
        (uint32_t)((((int64_t)b * a.hq + hq0 + g) * a.nsplit * kD + d) * sizeof(float));
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < nlive; s0 += kBatch) {
      u32x4 v[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int sp = s0 + i < nlive ? s0 + i : nlive - 1;
        v[i] = coh_ld16(a.part, base + (uint32_t)(sp * kD * sizeof(float)));
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        if (s0 + i < nlive) {
          s[0] += __uint_as_float(v[i].x);
          s[1] += __uint_as_float(v[i].y);
          s[2] += __uint_as_float(v[i].z);
          s[3] += __uint_as_float(v[i].w);
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float val = s[e];
      if (kF32) {
        const float gate = ((const float*)a.qkv)[(int64_t)b * a.ldq +
                                                 (int64_t)(hq0 + g) * 2 * kD + kD + d + e];
        val = val * (1.f / (1.f + expf(-gate)));
      }
      a.out[xp_off_g(b, (hq0 + g) * kD + d + e)] = f2bf(val);
    }
  }
  if (tid == 0) atomicExch(&a.counters[b * a.hkv + kvh], 0);
}

template <int kD, int kG, bool kF32>
int launch_gqa(const GqaArgs& a, int rows, hipStream_t s) {
  const dim3 grid(a.nsplit, a.hkv, rows);
  hipLaunchKernelGGL((k_gqa_scores<kD, kG, kF32>), grid, dim3(kBlock), 0, s, a);
  hipLaunchKernelGGL((k_gqa_pv<kD, kG, kF32>), grid, dim3(kBlock), 0, s, a);
  return launched("gqa_decode");
}

}  // namespace

extern "C" int tfd_gqa_decode(const TfdGqaArgs* args, void* stream) {
  if (!args) return fail(kBadArg, "gqa_decode: null args");
  const TfdGqaArgs& t = *args;
  const bool f32 = t.policy == TFD_POLICY_F32;
  if (t.policy != TFD_POLICY_F32 && t.policy != TFD_POLICY_BF16)
    return fail(kBadArg, "gqa_decode: policy %d", t.policy);
  if (!t.qkv || !t.pos || !t.page_table || !t.k_pool || !t.v_pool || !t.scores || !t.stats ||
      !t.part || !t.counters || !t.out ||
      (f32 && (!t.gamma_q || !t.gamma_k || !t.cos_table || !t.sin_table)))
    return fail(kBadArg, "gqa_decode: null pointer");
  const int D = t.head_dim;
  const int G = t.kv_heads > 0 ? t.heads / t.kv_heads : 0;
  const int qw = f32 ? 2 * D : D;
  if (t.rows <= 0 || t.rows > kMaxRowsG || t.kv_heads <= 0 || t.heads % t.kv_heads ||
      !((D == 128 && G == 4) || (D == 256 && G == 8)) ||
      t.ldq < t.heads * qw + 2 * t.kv_heads * D || t.max_pages <= 0 || t.num_pages <= 0 ||
      t.nsplit <= 0 || t.split_len < 0 || t.split_len > kMaxSplitLen ||
      t.split_len % kPage ||
      (int64_t)t.nsplit * (t.split_len > 0 ? t.split_len : kMaxSplitLen) <
          (int64_t)t.max_pages * kPage ||
      t.score_stride < t.max_pages * kPage ||
      (f32 && (t.rot_dim <= 0 || t.rot_dim % 2 || t.rot_dim > D || t.rope_rows <= 0)))
    return fail(kBadShape, "gqa_decode: rows=%d (1..32) heads=%d kv_heads=%d head_dim=%d "
                "(128 x4 or 256 x8) ldq=%d split_len=%d nsplit=%d stride=%d rot=%d", t.rows,
                t.heads, t.kv_heads, D, t.ldq, t.split_len, t.nsplit, t.score_stride, t.rot_dim);
  GqaArgs a;
  a.qkv = t.qkv;
  a.ldq = t.ldq;
  a.gamma_q = (const bf16*)t.gamma_q;
  a.gamma_k = (const bf16*)t.gamma_k;
  a.cos_t = (const bf16*)t.cos_table;
  a.sin_t = (const bf16*)t.sin_table;
  a.rope_rows = t.rope_rows;
  a.rot = t.rot_dim;
  a.pos = t.pos;
  a.table = t.page_table;
  a.max_pages = t.max_pages;
  a.kpool = (bf16*)t.k_pool;
  a.vpool = (bf16*)t.v_pool;
  a.num_pages = t.num_pages;
  a.hq = t.heads;
  a.hkv = t.kv_heads;
  a.scale = t.scale;
  a.eps = t.eps;
  a.scores = t.scores;
  a.sstride = t.score_stride;
  a.stats = t.stats;
  a.part = t.part;
  a.counters = t.counters;
  a.nsplit = t.nsplit;
  a.split_len = t.split_len;
  a.out = (bf16*)t.out;
  a.err = t.err;
  auto s = (hipStream_t)stream;
  if (D == 256) return f32 ? launch_gqa<256, 8, true>(a, t.rows, s)
                           : launch_gqa<256, 8, false>(a, t.rows, s);
  return f32 ? launch_gqa<128, 4, true>(a, t.rows, s) : launch_gqa<128, 4, false>(a, t.rows, s);
}
