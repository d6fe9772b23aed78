// Batched decode step (up to 32 sequences per step), bf16, for gfx950.
//
// The same HIR semantics as the batch-1 kernels (every matmul an f32 sum
// rounded once to bf16, the attention chain rounded where the HIR rounds), laid
// out for a batch: activations are [rows][n] row-major with explicit leading
// dimensions, every sequence has its own position and page-table row, and the
// projections are skinny GEMMs on the matrix cores (16x16x32 bf16 MFMA): at 32
// rows a projection is a real contraction (2 flops per weight byte per row), so
// the VALU dot path would be compute-bound before HBM is.
//
// Kernels of one layer (Qwen3-1.7B at batch 32):
//   rmsnorm_rows                 x -> bf16 normalised rows
//   gemm_skinny<STORE>           xn @ [q|k|v]^T            -> qkv   [B][HQ*D+2*HKV*D]
//   attn_rope_scores_batched     per (split, kv head, sequence), as the batch-1 phase
//   attn_pv_combine_batched      per (split, kv head, sequence), last block merges
//   gemm_skinny<RESID>           attn @ Wo^T + residual    -> h1
//   rmsnorm_rows, gemm_skinny<SWIGLU>, gemm_skinny<RESID> (down)
// and per step: rmsnorm_rows (final), gemm_skinny<LOGITS> (bf16-valued f32
// logits), argmax_rows, finalize_rows (pick, next token, position, embedding).

#include "decode_phases.h"
#include "host_common.h"
#include "tf_decode.h"

using namespace tfd;
using namespace tfd_host;

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxRows = 32;      // one skinny GEMM covers two 16-row MFMA tiles
constexpr int kSkSteps = 4;       // 32-wide k steps in flight per wave

// ---------------------------------------------------------------------------
// Row-wise RMSNorm (model.py:125-137 on each sequence's hidden state): one
// wave per row, the batch-1 arithmetic.
// ---------------------------------------------------------------------------
template <int kCmax>
__global__ __launch_bounds__(kWave) void k_rmsnorm_rows(const bf16* __restrict__ x, int ldx,
                                                        const bf16* __restrict__ gamma,
                                                        bf16* __restrict__ out, int ldo, int n,
                                                        float eps) {
  const int lane = threadIdx.x;
  const bf16* xr_p = x + (int64_t)blockIdx.x * ldx;
  bf16* o = out + (int64_t)blockIdx.x * ldo;
  u32x4 xr[kCmax];
  rms_norm_x<kCmax>(xr_p, gamma, n, eps, lane, xr);
  const int nch = n / 8;
#pragma unroll
  for (int i = 0; i < kCmax; ++i) {
    const int c = i * kWave + lane;
    if (c < nch) *reinterpret_cast<u32x4*>(o + (int64_t)c * 8) = xr[i];
  }
}

// ---------------------------------------------------------------------------
// Skinny GEMM: Y[m][n] = sum_k X[m][k] W[n][k] for m < M <= 32.
// A block owns one 16-column tile of Y (16 weight rows) for all rows; its four
// waves split K in quarters, each accumulating two 16x16 MFMA tiles (rows 0-15
// and 16-31) over 32-wide k steps, kSkSteps steps of loads in flight.  Operand
// layout of v_mfma_f32_16x16x32_bf16: lane l holds A[l % 16][8 (l / 16) .. +7],
// B[8 (l / 16) .. +7][l % 16], and gets D[4 (l / 16) .. +3][l % 16] -- so a lane
// loads 16 contiguous bytes of one weight row and of one activation row.  The
// quarters are summed in wave order through LDS; wave 0 applies the epilogue.
// ---------------------------------------------------------------------------
enum SkinnyEpi { kSkStore = 0, kSkResid = 1, kSkSwiglu = 2, kSkLogits = 3 };

template <int kEpi>
__global__ __launch_bounds__(kBlock) void k_gemm_skinny(const bf16* __restrict__ X, int ldx,
                                                        const bf16* __restrict__ W, int M, int K,
                                                        int N, const bf16* __restrict__ resid,
                                                        int ldr, void* __restrict__ out,
                                                        int ldo) {
  __shared__ f32x4 red[kWavesPerBlock][2][kWave];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int n0 = blockIdx.x * 16;
  const int r = lane & 15, kq = lane >> 4;
  const int nsteps = K / 32;
  const int per = (nsteps + kWavesPerBlock - 1) / kWavesPerBlock;
  const int s0 = wave * per;
  const int s1 = (s0 + per < nsteps) ? s0 + per : nsteps;
  // rows past M / N read row M-1 / N-1 (in bounds); their results are not stored
  const bf16* wrow = W + (int64_t)((n0 + r < N) ? n0 + r : N - 1) * K + 8 * kq;
  const bf16* xa = X + (int64_t)((r < M) ? r : M - 1) * ldx + 8 * kq;
  const bf16* xb = X + (int64_t)((16 + r < M) ? 16 + r : M - 1) * ldx + 8 * kq;
  f32x4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
  for (int s = s0; s < s1; s += kSkSteps) {
    u32x4 b[kSkSteps], a0[kSkSteps], a1[kSkSteps];
#pragma unroll
    for (int u = 0; u < kSkSteps; ++u) {
      const int k = ((s + u < s1) ? s + u : s1 - 1) * 32;
      b[u] = load16_stream(wrow + k);
      a0[u] = load16(xa + k);
      a1[u] = load16(xb + k);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kSkSteps; ++u) {
      if (s + u < s1) {
        const bf16x8_t bw = __builtin_bit_cast(bf16x8_t, b[u]);
        c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a0[u]), bw, c0,
                                                     0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a1[u]), bw, c1,
                                                     0, 0, 0);
      }
    }
  }
  red[wave][0][lane] = c0;
  red[wave][1][lane] = c1;
  __syncthreads();
  if (wave != 0) return;
  f32x4 t[2] = {red[0][0][lane], red[0][1][lane]};
#pragma unroll
  for (int w = 1; w < kWavesPerBlock; ++w) {
    const f32x4 u0 = red[w][0][lane], u1 = red[w][1][lane];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      t[0][e] += u0[e];
      t[1][e] += u1[e];
    }
  }
  const int n = n0 + r;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = 16 * h + 4 * kq + e;
      const float y = rbf(t[h][e]);
      if (kEpi == kSkSwiglu) {
        // gate at even columns, up at the odd column next to it (the next lane)
        const float u = __shfl_xor(y, 1, kWave);
        if ((r & 1) == 0 && m < M && n + 1 < N)
          ((bf16*)out)[(int64_t)m * ldo + n / 2] = f2bf(rbf(silu_f(y)) * u);
      } else if (m < M && n < N) {
        if (kEpi == kSkStore) {
          ((bf16*)out)[(int64_t)m * ldo + n] = f2bf(y);
        } else if (kEpi == kSkResid) {
          ((bf16*)out)[(int64_t)m * ldo + n] = f2bf(bf2f(resid[(int64_t)m * ldr + n]) + y);
        } else {
          ((float*)out)[(int64_t)m * ldo + n] = y;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Attention for a batch: grid (nsplit, kv heads, sequences); sequence b has its
// own position, page-table row, QKV row and workspaces.  The phase bodies are
// the batch-1 ones.
// ---------------------------------------------------------------------------
template <int D, int G>
__global__ __launch_bounds__(kBlock) void k_attn_scores_b(
    const bf16* __restrict__ qkv, int ldq, const bf16* __restrict__ gq,
    const bf16* __restrict__ gk, const bf16* __restrict__ cos_t, const bf16* __restrict__ sin_t,
    int rope_rows, const int* __restrict__ pos, const int* __restrict__ page_table, int max_pages,
    bf16* __restrict__ kpool, bf16* __restrict__ vpool, int num_pages, int kv_heads, float scale,
    float eps, float* __restrict__ S, int s_stride, float* __restrict__ smax,
    float* __restrict__ snew, int* err) {
  const int b = blockIdx.z, heads = kv_heads * G, nsplit = gridDim.x;
  const int P = coh_ldi(pos + b);
  const int* pt = page_table + (int64_t)b * max_pages;
  KTile<D> kt;
  k_tile_issue<D>(blockIdx.x, blockIdx.y, P, pt, max_pages, kpool, num_pages, kv_heads, kt);
  const QKPre pre = qk_prefetch<D, G>(P, P, gq, gk, cos_t, sin_t, rope_rows, pt, max_pages);
  __shared__ __attribute__((aligned(16))) uint32_t hs[(G + 2) * D / 2];
  stage_head<D, G>(blockIdx.y, heads, kv_heads, qkv + (int64_t)b * ldq, hs);
  __syncthreads();
  attn_scores_phase<D, G, false>(blockIdx.x, blockIdx.y, hs, pre, rope_rows, P, P, max_pages,
                                 kpool, vpool, num_pages, kv_heads, scale, eps,
                                 S + (int64_t)b * heads * s_stride, s_stride,
                                 smax + (int64_t)b * nsplit * heads, snew + (int64_t)b * heads,
                                 AttnLL{}, kt, err);
}

template <int D, int G>
__global__ __launch_bounds__(kBlock) void k_attn_pv_b(
    const bf16* __restrict__ qkv, int ldq, const int* __restrict__ pos,
    const int* __restrict__ page_table, int max_pages, const bf16* __restrict__ vpool,
    int num_pages, int kv_heads, const float* __restrict__ S, int s_stride,
    const float* __restrict__ smax, const float* __restrict__ snew, float* part_sum,
    float* part_out, int* counters, bf16* __restrict__ attn_out, int lda, int* err) {
  const int b = blockIdx.z, heads = kv_heads * G, nsplit = gridDim.x;
  int P = coh_ldi(pos + b);
  if (P < 0 || P >= max_pages * kPage) P = 0;
  const int* pt = page_table + (int64_t)b * max_pages;
  VTile<D> vt;
  v_tile_issue<D>(blockIdx.x, blockIdx.y, P, pt, max_pages, vpool, num_pages, kv_heads, vt);
  attn_pv_phase<D, G, false>(blockIdx.x, blockIdx.y, nsplit, qkv + (int64_t)b * ldq, P, pt,
                             max_pages, vpool, num_pages, kv_heads,
                             S + (int64_t)b * heads * s_stride, s_stride,
                             smax + (int64_t)b * nsplit * heads, snew + (int64_t)b * heads,
                             part_sum + (int64_t)b * nsplit * heads,
                             part_out + (int64_t)b * nsplit * heads * D,
                             counters + (int64_t)b * kv_heads, attn_out + (int64_t)b * lda,
                             AttnLL{}, vt, err);
}

// ---------------------------------------------------------------------------
// Greedy pick per row (generation.py:24-26: the first maximal bf16 logit) and
// the step's last node per sequence (the batch form of finalize_phase).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void k_argmax_rows(const float* __restrict__ logits, int ldl,
                                                      int V, int* __restrict__ pick) {
  const float* row = logits + (int64_t)blockIdx.x * ldl;
  float b = kNegInf;
  int i = 0x7fffffff;
  for (int k = threadIdx.x; k < V; k += blockDim.x) {
    const float v = row[k];
    if (better(v, k, b, i)) {
      b = v;
      i = k;
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ob = __shfl_xor(b, m, kWave);
    const int oi = __shfl_xor(i, m, kWave);
    if (better(ob, oi, b, i)) {
      b = ob;
      i = oi;
    }
  }
  __shared__ float sv[16];
  __shared__ int si[16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = b;
    si[wave] = i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float bb = sv[0];
    int ii = si[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w)
      if (better(sv[w], si[w], bb, ii)) {
        bb = sv[w];
        ii = si[w];
      }
    pick[blockIdx.x] = (ii >= 0 && ii < V) ? ii : 0;   // an all-NaN row has no pick
  }
}

__global__ __launch_bounds__(kBlock) void k_finalize_rows(
    const int* __restrict__ pick, const int* __restrict__ inp, int ld_inp,
    const int* __restrict__ plen, int64_t* __restrict__ ids, int* __restrict__ pos,
    int* __restrict__ sam, int ld_sam, int nsteps, const bf16* __restrict__ table,
    bf16* __restrict__ hid, int ldh, int hidden, int vocab, int* err) {
  const int b = blockIdx.x;
  __shared__ int next_s;
  if (threadIdx.x == 0) {
    const int p = pos[b];
    const int ii = pick[b];
    int next = ii;
    if (p < 0 || p >= nsteps) {
      raise_error(err, kErrStepRange);
    } else {
      sam[(int64_t)b * ld_sam + p] = ii;
      if (p + 1 < plen[b] && p + 1 < nsteps) next = inp[(int64_t)b * ld_inp + p + 1];
    }
    if (next < 0 || next >= vocab) {
      raise_error(err, kErrTokenRange);
      next = 0;
    }
    ids[b] = next;
    pos[b] = p + 1;
    next_s = next;
  }
  __syncthreads();
  const bf16* row = table + (int64_t)next_s * hidden;
  bf16* o = hid + (int64_t)b * ldh;
  for (int c = threadIdx.x; c < hidden / 8; c += kBlock)
    *reinterpret_cast<u32x4*>(o + (int64_t)c * 8) = load16(row + (int64_t)c * 8);
}

__global__ __launch_bounds__(kBlock) void k_embed_rows(const bf16* __restrict__ table,
                                                       const int64_t* __restrict__ ids,
                                                       bf16* __restrict__ out, int ldo,
                                                       int hidden, int vocab, int* err) {
  int64_t id = ids[blockIdx.x];
  if (id < 0 || id >= vocab) {
    if (threadIdx.x == 0) raise_error(err, kErrTokenRange);
    id = 0;
  }
  const bf16* row = table + id * (int64_t)hidden;
  bf16* o = out + (int64_t)blockIdx.x * ldo;
  for (int c = threadIdx.x; c < hidden / 8; c += kBlock)
    *reinterpret_cast<u32x4*>(o + (int64_t)c * 8) = load16(row + (int64_t)c * 8);
}

}  // namespace

#define TFD_ATTN_SWITCH_B(D, G, CALL)                                      \
  if (D == 128 && G == 2) { constexpr int kD = 128, kG = 2; CALL; }        \
  else if (D == 64 && G == 2) { constexpr int kD = 64, kG = 2; CALL; }     \
  else if (D == 128 && G == 1) { constexpr int kD = 128, kG = 1; CALL; }   \
  else return fail(kUnsupported, "attention: head_dim=%d group=%d not built", D, G);

extern "C" {

int tfd_rmsnorm_rows_bf16(const void* x, int ldx, const void* gamma, void* out, int ldo,
                          int rows, int n, float eps, void* stream) {
  if (!x || !gamma || !out) return fail(kBadArg, "rmsnorm_rows: null pointer");
  if (rows <= 0 || n <= 0 || n % 8 || ldx < n || ldo < n || ldx % 8 || ldo % 8)
    return fail(kBadShape, "rmsnorm_rows: rows=%d n=%d ldx=%d ldo=%d", rows, n, ldx, ldo);
  auto s = (hipStream_t)stream;
  TFD_CMAX_SWITCH(n, hipLaunchKernelGGL((k_rmsnorm_rows<kC>), dim3(rows), dim3(kWave), 0, s,
                                        (const bf16*)x, ldx, (const bf16*)gamma, (bf16*)out, ldo,
                                        n, eps));
  return launched("rmsnorm_rows");
}

int tfd_gemm_skinny_bf16(const void* x, int ldx, const void* w, int M, int K, int N,
                         int epilogue, const void* resid, int ldr, void* out, int ldo,
                         void* stream) {
  if (!x || !w || !out) return fail(kBadArg, "gemm_skinny: null pointer");
  if (M <= 0 || M > kMaxRows || K <= 0 || K % 32 || N <= 0 || ldx < K || ldx % 8)
    return fail(kBadShape, "gemm_skinny: M=%d (1..32) K=%d (multiple of 32) N=%d ldx=%d", M, K,
                N, ldx);
  if (epilogue == TFD_EPI_RESID && (!resid || ldr < N))
    return fail(kBadArg, "gemm_skinny: residual epilogue needs resid with ldr >= N");
  if (epilogue == TFD_EPI_SWIGLU ? (N % 2 || ldo < N / 2) : ldo < N)
    return fail(kBadShape, "gemm_skinny: ldo=%d too small for N=%d", ldo, N);
  const dim3 grid((N + 15) / 16);
  auto s = (hipStream_t)stream;
  auto xb = (const bf16*)x;
  auto wb = (const bf16*)w;
  auto rb = (const bf16*)resid;
  switch (epilogue) {
    case TFD_EPI_STORE:
      hipLaunchKernelGGL(k_gemm_skinny<kSkStore>, grid, dim3(kBlock), 0, s, xb, ldx, wb, M, K, N,
                         rb, ldr, out, ldo);
      break;
    case TFD_EPI_RESID:
      hipLaunchKernelGGL(k_gemm_skinny<kSkResid>, grid, dim3(kBlock), 0, s, xb, ldx, wb, M, K, N,
                         rb, ldr, out, ldo);
      break;
    case TFD_EPI_SWIGLU:
      hipLaunchKernelGGL(k_gemm_skinny<kSkSwiglu>, grid, dim3(kBlock), 0, s, xb, ldx, wb, M, K,
                         N, rb, ldr, out, ldo);
      break;
    case TFD_EPI_LOGITS:
      hipLaunchKernelGGL(k_gemm_skinny<kSkLogits>, grid, dim3(kBlock), 0, s, xb, ldx, wb, M, K,
                         N, rb, ldr, out, ldo);
      break;
    default:
      return fail(kBadArg, "gemm_skinny: epilogue %d", epilogue);
  }
  return launched("gemm_skinny");
}

int tfd_attn_rope_scores_paged_batched(
    const void* qkv, int ldq, const void* gamma_q, const void* gamma_k, const void* cos_table,
    const void* sin_table, int rope_rows, const int32_t* pos, const int32_t* page_table,
    int max_pages, void* k_pool, void* v_pool, int num_pages, int batch, int heads, int kv_heads,
    int head_dim, float scale, float eps, float* scores, int score_stride, float* split_max,
    float* score_new, int nsplit, int32_t* err, void* stream) {
  if (!qkv || !gamma_q || !gamma_k || !cos_table || !sin_table || !pos || !page_table ||
      !k_pool || !v_pool || !scores || !split_max || !score_new)
    return fail(kBadArg, "attn_rope_scores_batched: null pointer");
  if (batch <= 0 || batch > 65535 || kv_heads <= 0 || heads % kv_heads || nsplit <= 0 ||
      max_pages <= 0 || num_pages <= 0)
    return fail(kBadShape, "attn_rope_scores_batched: batch=%d heads=%d kv_heads=%d nsplit=%d",
                batch, heads, kv_heads, nsplit);
  if ((int64_t)nsplit * kSplit < (int64_t)max_pages * kPage || score_stride < nsplit * kSplit ||
      ldq < (heads + 2 * kv_heads) * head_dim)
    return fail(kBadShape, "attn_rope_scores_batched: nsplit=%d / score_stride=%d / ldq=%d do "
                "not cover the cache", nsplit, score_stride, ldq);
  const int G = heads / kv_heads;
  const dim3 grid(nsplit, kv_heads, batch);
  auto s = (hipStream_t)stream;
  TFD_ATTN_SWITCH_B(head_dim, G,
      hipLaunchKernelGGL((k_attn_scores_b<kD, kG>), grid, dim3(kBlock), 0, s, (const bf16*)qkv,
                         ldq, (const bf16*)gamma_q, (const bf16*)gamma_k,
                         (const bf16*)cos_table, (const bf16*)sin_table, rope_rows, pos,
                         page_table, max_pages, (bf16*)k_pool, (bf16*)v_pool, num_pages,
                         kv_heads, scale, eps, scores, score_stride, split_max, score_new, err));
  return launched("attn_rope_scores_batched");
}

int tfd_attn_pv_combine_paged_batched(
    const void* qkv, int ldq, const int32_t* pos, const int32_t* page_table, int max_pages,
    const void* v_pool, int num_pages, int batch, int heads, int kv_heads, int head_dim,
    const float* scores, int score_stride, const float* split_max, const float* score_new,
    float* part_sum, float* part_out, int nsplit, int32_t* counters, void* attn_out, int lda,
    int32_t* err, void* stream) {
  if (!qkv || !pos || !page_table || !v_pool || !scores || !split_max || !score_new ||
      !part_sum || !part_out || !counters || !attn_out)
    return fail(kBadArg, "attn_pv_combine_batched: null pointer");
  if (batch <= 0 || batch > 65535 || kv_heads <= 0 || heads % kv_heads || nsplit <= 0 ||
      max_pages <= 0 || num_pages <= 0 || lda < heads * head_dim)
    return fail(kBadShape, "attn_pv_combine_batched: batch=%d heads=%d kv_heads=%d nsplit=%d "
                "lda=%d", batch, heads, kv_heads, nsplit, lda);
  if ((int64_t)nsplit * kSplit < (int64_t)max_pages * kPage || score_stride < nsplit * kSplit)
    return fail(kBadShape, "attn_pv_combine_batched: nsplit=%d does not cover the cache", nsplit);
  const int G = heads / kv_heads;
  const dim3 grid(nsplit, kv_heads, batch);
  auto s = (hipStream_t)stream;
  TFD_ATTN_SWITCH_B(head_dim, G,
      hipLaunchKernelGGL((k_attn_pv_b<kD, kG>), grid, dim3(kBlock), 0, s, (const bf16*)qkv, ldq,
                         pos, page_table, max_pages, (const bf16*)v_pool, num_pages, kv_heads,
                         scores, score_stride, split_max, score_new, part_sum, part_out,
                         counters, (bf16*)attn_out, lda, err));
  return launched("attn_pv_combine_batched");
}

int tfd_argmax_rows(const float* logits, int ldl, int rows, int vocab, int32_t* pick,
                    void* stream) {
  if (!logits || !pick) return fail(kBadArg, "argmax_rows: null pointer");
  if (rows <= 0 || vocab <= 0 || ldl < vocab)
    return fail(kBadShape, "argmax_rows: rows=%d vocab=%d ldl=%d", rows, vocab, ldl);
  hipLaunchKernelGGL(k_argmax_rows, dim3(rows), dim3(1024), 0, (hipStream_t)stream, logits, ldl,
                     vocab, pick);
  return launched("argmax_rows");
}

int tfd_finalize_rows(const int32_t* pick, int rows, const int32_t* inp, int ld_inp,
                      const int32_t* prompt_len, int64_t* ids, int32_t* pos, int32_t* sam,
                      int ld_sam, int nsteps, const void* table, void* hid, int ldh, int hidden,
                      int vocab, int32_t* err, void* stream) {
  if (!pick || !inp || !prompt_len || !ids || !pos || !sam || !table || !hid)
    return fail(kBadArg, "finalize_rows: null pointer");
  if (rows <= 0 || nsteps <= 0 || ld_inp < nsteps || ld_sam < nsteps || hidden <= 0 ||
      hidden % 8 || ldh < hidden || ldh % 8 || vocab <= 0)
    return fail(kBadShape, "finalize_rows: rows=%d nsteps=%d hidden=%d ldh=%d", rows, nsteps,
                hidden, ldh);
  hipLaunchKernelGGL(k_finalize_rows, dim3(rows), dim3(kBlock), 0, (hipStream_t)stream, pick,
                     inp, ld_inp, prompt_len, ids, pos, sam, ld_sam, nsteps, (const bf16*)table,
                     (bf16*)hid, ldh, hidden, vocab, err);
  return launched("finalize_rows");
}

int tfd_embed_rows_bf16(const void* table, const int64_t* ids, void* out, int ldo, int rows,
                        int hidden, int vocab, int32_t* err, void* stream) {
  if (!table || !ids || !out) return fail(kBadArg, "embed_rows: null pointer");
  if (rows <= 0 || hidden <= 0 || hidden % 8 || ldo < hidden || ldo % 8 || vocab <= 0)
    return fail(kBadShape, "embed_rows: rows=%d hidden=%d ldo=%d", rows, hidden, ldo);
  hipLaunchKernelGGL(k_embed_rows, dim3(rows), dim3(kBlock), 0, (hipStream_t)stream,
                     (const bf16*)table, ids, (bf16*)out, ldo, hidden, vocab, err);
  return launched("embed_rows");
}

}  // extern "C"
