// Chunked KDN memory scan (shared by iso_kdn and diag_kdn), forward and backward.
//
// Recurrence per (b, h):  S_hat = diag(alpha_t) S;  delta = v_t - k_t^T S_hat;
//                         S = S_hat + kappa_t delta^T;  o_t = scale q_t^T S
// (iso: kappa_t = beta_t k_t).  Reference: lit_gpt/kdn_ops/iso_kdn_naive.py:449-533 and
// diag_kdn_naive.py:570-655 (chunk form), diag_kdn_chunk.py:720-1861 (production kernels).
//
// Chunk of C = 64 tokens, g = natural-log chunk-local cumulative gate (g_cumsum * ln 2);
// the returned dg is the cotangent in these natural-log coordinates (not reverse-summed):
//   N[c,s] = sum_i k_ci kappa_si e^{g_ci - g_si}   (s < c)       (write interactions)
//   M[c,s] = scale sum_i q_ci kappa_si e^{g_ci - g_si}   (s <= c) (readout interactions)
//   U = (I+N)^-1 V,  W = (I+N)^-1 (K e^g),  Kf = kappa e^{g_last - g},  Qg = scale Q e^g
//   delta = U - W S_0,  O = Qg S_0 + M delta,  S_C = e^{g_last} S_0 + Kf^T delta
//
// Kernels (grid = one workgroup per chunk unless noted, 256 threads = 4 waves):
//   intra_fwd    N/M (MFMA, one anchor per chunk, then one per 16-token block for the chunks
//                that need it), forward substitution for U, W; Kf, Qg
//   state_fwd    serial over chunks, one workgroup per (V-slice, b, h): h per chunk, delta
//   readout      chunk-parallel O = Qg h + M delta (kdn_state.h)
//   state_bwd    serial reverse (kdn_state.h): d delta = M^T dO + Kf dS;  dS <- e dS + Qg^T dO - W^T d delta
//   chunk_bwd    (kdn_bwd.h, 512 threads) per chunk: dQg = dO h^T, dW = -d delta h^T, dKf = delta dh^T,
//                dM = dO delta^T, g_last terms; dV = (I+N)^-T d delta, dKg = (I+N)^-T dW,
//                dN = -(dV U^T + dKg W^T); dq, dk, dkappa (or dbeta), dg from dN, dM and the
//                elementwise factors
//   *_exact      the chunks the forward flagged: the same backward by per-block anchors and scalar
//                substitution (the products above come from chunk_bwd through HBM)
//
// g is kept in the base-2 units of g_cumsum, so e^{g_c - g_s} = exp2(G_c - G_s).
// Decay factors (c >= s) are split at the start a of the row block (16 tokens):
// exp2(G_c - G_a) exp2(G_a - G_s).  Off-diagonal blocks have both factors <= 1 for
// non-increasing G.  Diagonal blocks use the split only when the block's decay span
// is <= 86 (base 2, no overflow); otherwise an exact per-element path runs.
// Products use fp32 MFMA (v_mfma_f32_16x16x4_f32), fp32 accumulate.
#include <mutex>

#include "kdn_common.h"
#include "kdn_state.h"
#include "kdn_intra.h"
#include "kdn_bwd.h"
#include "../../include/kdn.h"

namespace {

constexpr int C = 64;        // chunk length
constexpr int NS = C + 4;    // LDS row stride of C x C tiles
constexpr float kSpanMax = 86.f;  // base-2 units: 2^86 ~ 8e25 leaves headroom below FLT_MAX

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ int64_t bthk(int b, int t, int h, int i, int T, int H, int D) {
  return (((int64_t)b * T + t) * H + h) * D + i;
}
// [B,H,T,D] row offset for (bh, t)
__device__ __forceinline__ int64_t bht(int bh, int t, int T, int D) { return ((int64_t)bh * T + t) * D; }

// ---------------------------------------------------------------------------
// Chunk staging: k, kappa, g (natural) and optionally q into LDS as fp32 [C][K+4].
// Rows >= L are zero; g rows >= L repeat row L-1.  Also the per-block decay spans.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float lds_f(const float* p, int i) { return p[i]; }
__device__ __forceinline__ float lds_f(const bf16_t* p, int i) { return bf2f(p[i]); }

// Copy a [ROWS x D] fp32 tile (row r at src + r * stride; rows >= L read as zero) into LDS
// dst[r * DP + col] with 16-byte loads, all issued before any store.
template <int ROWS, int D, int DP>
__device__ __forceinline__ void stage_f32(const float* __restrict__ src, int64_t stride, int L, float* dst) {
  constexpr int D4 = D / 4, N4 = ROWS * D4, PER = (N4 + 255) / 256;
  static_assert(DP % 4 == 0, "16-byte aligned LDS rows");
  float4 v[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int e = threadIdx.x + 256 * u, r = e / D4, c4 = e % D4;
    v[u] = (e < N4 && r < L) ? *reinterpret_cast<const float4*>(src + r * stride + 4 * c4) : float4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int e = threadIdx.x + 256 * u, r = e / D4, c4 = e % D4;
    if (e < N4) *reinterpret_cast<float4*>(dst + r * DP + 4 * c4) = v[u];
  }
}

// Copy a [ROWS x D] bf16 tile into LDS as fp32 (DP % 4 == 0) or as bf16 (DP % 8 == 0).
template <int ROWS, int D, int DP, typename TD>
__device__ __forceinline__ void stage_bf16(const bf16_t* __restrict__ src, int64_t stride, int L, TD* dst) {
  constexpr int D8 = D / 8, N8 = ROWS * D8, PER = (N8 + 255) / 256;
  uint4 v[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int e = threadIdx.x + 256 * u, r = e / D8, c8 = e % D8;
    v[u] = (e < N8 && r < L) ? *reinterpret_cast<const uint4*>(src + r * stride + 8 * c8) : uint4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int e = threadIdx.x + 256 * u, r = e / D8, c8 = e % D8;
    if (e >= N8) continue;
    if constexpr (sizeof(TD) == 2) {
      static_assert(DP % 8 == 0, "16-byte aligned LDS rows");
      *reinterpret_cast<uint4*>(dst + r * DP + 8 * c8) = v[u];
    } else {
      static_assert(DP % 4 == 0, "16-byte aligned LDS rows");
      const uint32_t w4[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
      float f[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f[2 * q] = __uint_as_float(w4[q] << 16);
        f[2 * q + 1] = __uint_as_float(w4[q] & 0xffff0000u);
      }
      *reinterpret_cast<float4*>(dst + r * DP + 8 * c8) = float4{f[0], f[1], f[2], f[3]};
      *reinterpret_cast<float4*>(dst + r * DP + 8 * c8 + 4) = float4{f[4], f[5], f[6], f[7]};
    }
  }
}

// LDS row stride of the staged q / k arrays: K + 4 floats or K + 8 bf16 (16-byte rows).
template <int K, typename TQK>
struct QKStride {
  static constexpr int value = sizeof(TQK) == 2 ? K + 8 : K + 4;
};

// In-op L2 norm of a staged chunk of raw q or k rows (L rows, LDS stride KQ): with rs_out each row's
// rstd is computed (sum of squares in the order of l2norm_fwd_vec_kernel) and written to rs_out,
// else it is read from rs_in ([B,T,H], row c of the chunk at row0 + c H).  The staged values become
// the scan's operand y = bf16(x rstd).  Ends with a barrier.
template <int K, typename TQK>
__device__ void l2n_staged(TQK* sX, int L, int64_t row0, int H, const float* __restrict__ rs_in,
                           float* __restrict__ rs_out, float* sRs) {
  constexpr int KQ = QKStride<K, TQK>::value;
  const int tid = threadIdx.x;
  if (tid < L) {
    float rs;
    if (rs_out) {
      float S[K / 8];
#pragma unroll
      for (int r = 0; r < K / 8; ++r) {
        float x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = lds_f(sX, tid * KQ + 8 * r + j);
        S[r] = l2n_run(x);
      }
      rs = l2n_rstd(l2n_tree<K / 8>(S));
      rs_out[row0 + (int64_t)tid * H] = rs;
    } else {
      rs = rs_in[row0 + (int64_t)tid * H];
    }
    sRs[tid] = rs;
  }
  __syncthreads();
  for (int e = tid; e < L * K; e += 256) {
    const int c = e / K, i = e - c * K;
    const float y = l2n(lds_f(sX, c * KQ + i), sRs[c]);
    if constexpr (sizeof(TQK) == 2) sX[c * KQ + i] = f2bf(y);
    else sX[c * KQ + i] = y;
  }
  __syncthreads();
}

// Stage a chunk's g, kappa, k and (sQ non-null) q rows.  With the in-op L2 norm (iso scan) q and k
// are raw: the forward (rs_out) normalises them and writes their rows' rstd, the backward (rs_in)
// normalises them with the forward's.
template <int K, bool ISO, typename TQK>
__device__ void stage_chunk(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const float* __restrict__ kap,
                            const float* __restrict__ gc, int b, int h, int T, int H, int t0, int L, TQK* sQ,
                            TQK* sK, float* sA, float* sG, float* sSpan, const float* q_rs_in = nullptr,
                            const float* k_rs_in = nullptr, float* q_rs_out = nullptr, float* k_rs_out = nullptr) {
  constexpr int KP = K + 4;
  constexpr int KQ = QKStride<K, TQK>::value;
  const int tid = threadIdx.x;
  const int64_t base = (((int64_t)b * T + t0) * H + h) * K, stride = (int64_t)H * K;
  stage_f32<C, K, KP>(gc + base, stride, L, sG);  // base-2 chunk-local prefix
  if (!ISO) stage_f32<C, K, KP>(kap + base, stride, L, sA);
  stage_bf16<C, K, KQ>(k + base, stride, L, sK);
  if (sQ) stage_bf16<C, K, KQ>(q + base, stride, L, sQ);
  __syncthreads();
  if (k_rs_in || k_rs_out) {
    __shared__ float sRs[C];
    const int64_t row0 = ((int64_t)b * T + t0) * H + h;
    l2n_staged<K, TQK>(sK, L, row0, H, k_rs_in, k_rs_out, sRs);
    if (sQ) l2n_staged<K, TQK>(sQ, L, row0, H, q_rs_in, q_rs_out, sRs);
  }
  if (ISO) {  // kappa = beta k
    for (int e = tid; e < C * K; e += 256) {
      const int c = e / K, i = e - c * K;
      sA[c * KP + i] = c < L ? kap[((int64_t)b * T + t0 + c) * H + h] * lds_f(sK, c * KQ + i) : 0.f;
    }
  }
  if (L < C) {  // g rows past the end repeat the last token's prefix
    for (int e = tid; e < (C - L) * K; e += 256) {
      const int c = L + e / K, i = e % K;
      sG[c * KP + i] = sG[(L - 1) * KP + i];
    }
  }
  __syncthreads();
  // span of block w (= wave w): max_i,r |g[16w][i] - g[16w + r][i]|
  {
    const int w = tid >> 6, lane = tid & 63;
    float m = 0.f;
    for (int i = lane; i < K; i += 64) {
      const float ga = sG[(16 * w) * KP + i];
      for (int r = 1; r < 16; ++r) m = fmaxf(m, fabsf(ga - sG[(16 * w + r) * KP + i]));
    }
    m = wave_max(m);
    if (lane == 0) sSpan[w] = m;
  }
  __syncthreads();
}

// Lower 16x16 tile list (I, J), J <= I, in an order that balances the 4 waves.
__device__ __forceinline__ void lower_tile(int t, int& I, int& J) {
  // 0:(0,0) 1:(1,1) 2:(2,2) 3:(3,3) 4:(1,0) 5:(2,1) 6:(3,2) 7:(2,0) 8:(3,1) 9:(3,0), 2-bit packed
  I = (0xfb9e4u >> (2 * t)) & 3;
  J = (0x124e4u >> (2 * t)) & 3;
}

// Build N (strictly lower, into sN [C][NS], or its transpose) and optionally M (lower incl.
// diagonal, scaled, written to global gM [C][C], zeros above the diagonal).
template <int K, bool WITH_M, bool N_TRANSPOSED>
__device__ void build_NM(const float* sQ, const float* sK, const float* sA, const float* sG, const float* sSpan,
                         float scale, float* sN, float* __restrict__ gM) {
  constexpr int KP = K + 4;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // upper tiles -> zero
  for (int e = tid; e < 6 * 256; e += 256) {
    const int ut = e >> 8, r = (e >> 4) & 15, cc = e & 15;
    // upper tiles (0,1) (0,2) (0,3) (1,2) (1,3) (2,3), 2-bit packed
    const int c = 16 * ((0x940u >> (2 * ut)) & 3) + r, s = 16 * ((0xfb9u >> (2 * ut)) & 3) + cc;
    sN[N_TRANSPOSED ? s * NS + c : c * NS + s] = 0.f;
    if (WITH_M) gM[c * C + s] = 0.f;
  }
  for (int t = w; t < 10; t += 4) {
    int I, J;
    lower_tile(t, I, J);
    const int a = 16 * I;
    const bool diag = I == J;
    const bool fast = !diag || sSpan[I] <= kSpanMax;
    f32x4 accN = zero4(), accM = zero4();
    if (fast) {
      const int cA = a + (lane & 15), sB = 16 * J + (lane & 15);
#pragma unroll 4
      for (int st = 0; st < K / 4; ++st) {
        const int i = 4 * st + (lane >> 4);
        const float ga = sG[a * KP + i];
        const float el = exp2f(sG[cA * KP + i] - ga);
        const float br = sA[sB * KP + i] * exp2f(ga - sG[sB * KP + i]);
        accN = mfma4(sK[cA * KP + i] * el, br, accN);
        if (WITH_M) accM = mfma4(sQ[cA * KP + i] * el, br, accM);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = a + 4 * (lane >> 4) + j, s = 16 * J + (lane & 15);
      float nv = accN[j], mv = accM[j];
      if (!fast) {
        nv = 0.f;
        mv = 0.f;
        if (s <= c) {
          for (int i = 0; i < K; ++i) {
            const float tv = sA[s * KP + i] * exp2f(sG[c * KP + i] - sG[s * KP + i]);
            nv += sK[c * KP + i] * tv;
            if (WITH_M) mv += sQ[c * KP + i] * tv;
          }
        }
      }
      if (diag) {
        if (s >= c) nv = 0.f;
        if (s > c) mv = 0.f;
      }
      sN[N_TRANSPOSED ? s * NS + c : c * NS + s] = nv;
      if (WITH_M) gM[c * C + s] = mv * scale;
    }
  }
}

// ===========================================================================
// Forward intra-chunk kernel.
// ===========================================================================
// Exact path for one chunk (per-block decay anchors, per-element diagonal blocks when a
// block's span exceeds kSpanMax, scalar forward substitution).  Runs only for the chunks the
// MFMA kernels (kdn_intra.h) leave flagged: a 16-token block spans more than their block-anchor range.
// lds: ExactFwdLds<K, V>::bytes of a caller's 16-byte aligned pool.
template <int K, int V>
struct ExactFwdLds {
  static constexpr int KP = K + 4, XP = V + K + 4;
  static constexpr int OFF2 = (2 * C * KP > C * XP) ? 2 * C * KP : C * XP;
  static constexpr int bytes = (OFF2 + 2 * C * KP + C * NS + 4) * 4;
};
template <int K, int V, bool ISO>
__device__ void intra_fwd_exact_chunk(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const float* __restrict__ kap,
    const bf16_t* __restrict__ v, const float* __restrict__ gc, int T, int H, int NT, float scale,
    float* __restrict__ U, float* __restrict__ W, float* __restrict__ Kf, float* __restrict__ Qg,
    float* __restrict__ Mg, float* __restrict__ Ag, int n, int bh, float* __restrict__ q_rstd,
    float* __restrict__ k_rstd, unsigned char* lds) {
  constexpr int KP = K + 4;
  constexpr int XP = V + K + 4;
  // sQ | sA are dead after Kf / Qg are written and are then reused for the solve's sX [C][XP]
  constexpr int OFF2 = ExactFwdLds<K, V>::OFF2;
  float* sBuf = reinterpret_cast<float*>(lds);
  float* sN = sBuf + OFF2 + 2 * C * KP;  // transposed: sN[s * NS + c] = N[c][s]
  float* sSpan = sN + C * NS;
  float* sQ = sBuf;
  float* sA = sBuf + C * KP;
  float* sK = sBuf + OFF2;
  float* sG = sBuf + OFF2 + C * KP;
  float* sX = sBuf;
  const int b = bh / H, h = bh % H;
  const int t0 = n * C, L = min(C, T - t0);
  const int tid = threadIdx.x;
  stage_chunk<K, ISO, float>(q, k, kap, gc, b, h, T, H, t0, L, sQ, sK, sA, sG, sSpan, nullptr, nullptr, q_rstd,
                             k_rstd);
  build_NM<K, true, true>(sQ, sK, sA, sG, sSpan, scale, sN, Mg + ((int64_t)bh * NT + n) * C * C);
  // Kf = kappa e^{g_last - g};  Qg = scale q e^g
  if (tid < 2 * K) {
    const int i = tid % K;
    const bool isKf = tid < K;
    const float gl = sG[(L - 1) * KP + i];
    for (int c = 0; c < L; ++c) {
      const int64_t o = bht(bh, t0 + c, T, K) + i;
      if (isKf) Kf[o] = sA[c * KP + i] * exp2f(gl - sG[c * KP + i]);
      else Qg[o] = scale * sQ[c * KP + i] * exp2f(sG[c * KP + i]);
    }
  }
  __syncthreads();
  // forward substitution (I+N) X = [V | K e^g], thread = column; 16-row blocks
  if (tid < V + K) {
    const int j = tid;
    const bool isV = j < V;
    const int col = isV ? j : j - V;
    float* dst = isV ? U : W;
    const int D = isV ? V : K;
#pragma unroll 1
    for (int I = 0; I < 4; ++I) {
      float acc[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int c = 16 * I + r;
        float x = 0.f;
        if (c < L) x = isV ? bf2f(v[bthk(b, t0 + c, h, col, T, H, V)]) : sK[c * KP + col] * exp2f(sG[c * KP + col]);
        acc[r] = x;
      }
#pragma unroll 1
      for (int s = 0; s < 16 * I; ++s) {
        const float xs = sX[s * XP + j];
        const float4* nrow = reinterpret_cast<const float4*>(sN + s * NS + 16 * I);
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const float4 nv = nrow[r4];
          acc[4 * r4 + 0] -= nv.x * xs;
          acc[4 * r4 + 1] -= nv.y * xs;
          acc[4 * r4 + 2] -= nv.z * xs;
          acc[4 * r4 + 3] -= nv.w * xs;
        }
      }
#pragma unroll
      for (int r = 1; r < 16; ++r) {
#pragma unroll
        for (int r2 = 0; r2 < r; ++r2) acc[r] -= sN[(16 * I + r2) * NS + 16 * I + r] * acc[r2];
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int c = 16 * I + r;
        sX[c * XP + j] = acc[r];
        if (c < L) dst[bht(bh, t0 + c, T, D) + col] = acc[r];
      }
    }
  }
}

// Grid-stride pass over the chunks the MFMA kernel flagged (flags[chunk] != 0).
// True in every thread when any chunk of this workgroup's grid-stride share (blockIdx.x,
// blockIdx.x + gridDim.x, ...) is flagged.  One flag per thread, loaded in parallel, so a
// workgroup with nothing to do exits after one load instead of one dependent load per chunk.
__device__ __forceinline__ bool any_flagged(const int* __restrict__ flags, int NB) {
  int any = 0;
  for (int lin = blockIdx.x + threadIdx.x * gridDim.x; lin < NB; lin += blockDim.x * gridDim.x) any |= flags[lin];
  return __syncthreads_or(any) != 0;
}

// The chunks intra_fwd_kernel flagged, of chunks n0 .. n1 - 1 of every head (the forward's schedule may build a
// sequence in two ranges), grid-stride (i = blockIdx.x, + gridDim.x, ...: head i / len, chunk n0 + i % len).
// Each flagged chunk takes the block-anchor path, and the exact path when that leaves it flagged, in the same
// workgroup; the two paths' LDS arrays share one pool (one workgroup per CU).  A workgroup first loads all its
// chunks' flags at once and exits when none is set.  One launch for both paths.
template <int K, int V, bool ISO, bool NORM>
__global__ __launch_bounds__(256) void intra_fwd_flagged_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const float* __restrict__ kap,
    const bf16_t* __restrict__ v, const float* __restrict__ gc, int T, int H, int NT, int BH, int n0, int n1,
    float scale, float* __restrict__ U, float* __restrict__ W, float* __restrict__ Kf, float* __restrict__ Qg,
    float* __restrict__ Mg, float* __restrict__ Ag, int* __restrict__ flags, float* __restrict__ q_rstd,
    float* __restrict__ k_rstd) {
  constexpr int LB = kdn_intra::BlockLds<K, V>::bytes, LE = ExactFwdLds<K, V>::bytes;
  __shared__ __attribute__((aligned(16))) unsigned char lds[LB > LE ? LB : LE];
  const int len = n1 - n0, N = BH * len;
  int any = 0;
  for (int i = blockIdx.x + threadIdx.x * gridDim.x; i < N; i += blockDim.x * gridDim.x)
    any |= flags[(int64_t)(i / len) * NT + n0 + i % len];
  if (__syncthreads_or(any) == 0) return;
  for (int i = blockIdx.x; i < N; i += gridDim.x) {
    const int bh = i / len, n = n0 + i % len;
    if (flags[(int64_t)bh * NT + n] == 0) continue;
    __syncthreads();  // LDS of the previous chunk is dead
    if (!kdn_intra::intra_fwd_block_chunk<K, V, ISO, NORM>(q, k, kap, v, gc, T, H, NT, scale, U, W, Kf, Qg, Mg, Ag,
                                                           flags, q_rstd, k_rstd, n, bh, lds)) {
      __syncthreads();  // the block path's span reads are done
      intra_fwd_exact_chunk<K, V, ISO>(q, k, kap, v, gc, T, H, NT, scale, U, W, Kf, Qg, Mg, Ag, n, bh, q_rstd, k_rstd,
                                       lds);
    }
  }
}

// ===========================================================================
// Backward: transposed triangular solves and dN.
// ===========================================================================
// LDS bytes of the two exact backward steps (their arrays are carved from a caller's 16-byte aligned pool,
// so one kernel can run both on the same bytes).  Every array size is a multiple of 4 floats.
template <int K, int V>
struct ExactLds {
  static constexpr int KP = K + 4, XP = V + K + 4, P1 = 3 * C * KP, P2 = 2 * C * XP, R1 = P1 > P2 ? P1 : P2;
  static constexpr int KQ = K + 8;  // QKStride<K, bf16_t>
  static constexpr int solve = (R1 + C * NS + 4) * 4;
  static constexpr int contrib = 2 * C * KQ * 2 + (2 * C * KP + 2 * C * NS + 4 + 5 * K + C * (K / 16)) * 4;
  static constexpr int both = solve > contrib ? solve : contrib;
};

// Exact path for one chunk (rebuilds N with per-block anchors, scalar back substitution); runs
// only for the chunks the forward flagged as outside the single-anchor range.  lds: ExactLds::solve bytes.
template <int K, int V, bool ISO>
__device__ void bwd_solve_exact_chunk(
    const bf16_t* __restrict__ k, const float* __restrict__ kap, const float* __restrict__ gc,
    const float* __restrict__ dDl, const float* __restrict__ dWg, const float* __restrict__ U,
    const float* __restrict__ W, int T, int H, int NT, bf16_t* __restrict__ dv, float* __restrict__ dKg,
    float* __restrict__ dNg, int n, int bh, const float* __restrict__ k_rstd, bool dd16, unsigned char* lds) {
  constexpr int KP = K + 4;
  constexpr int XP = V + K + 4;
  // phase 1: sK | sA | sG (3 x C x KP); phase 2 (after the solve) reuses it as sX | sUW (2 x C x XP)
  constexpr int R1 = ExactLds<K, V>::R1;
  float* sBuf = reinterpret_cast<float*>(lds);
  float* sN = sBuf + R1;
  float* sSpan = sN + C * NS;
  float* sK = sBuf;
  float* sA = sBuf + C * KP;
  float* sG = sBuf + 2 * C * KP;
  const int b = bh / H, h = bh % H;
  const int t0 = n * C, L = min(C, T - t0);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  stage_chunk<K, ISO, float>(nullptr, k, kap, gc, b, h, T, H, t0, L, (float*)nullptr, sK, sA, sG, sSpan, nullptr,
                             k_rstd);
  build_NM<K, false, false>(nullptr, sK, sA, sG, sSpan, 0.f, sN, nullptr);
  __syncthreads();  // sK / sA / sG are dead from here on; sX reuses their space
  float* sX = sBuf;
  float* sUW = sBuf + C * XP;
  // back substitution (I+N)^T X = [d delta | dW], thread = column; 16-row blocks, last first
  if (tid < V + K) {
    const int j = tid;
    const bool isV = j < V;
    const int col = isV ? j : j - V;
#pragma unroll 1
    for (int I = 3; I >= 0; --I) {
      float acc[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int c = 16 * I + r;
        float x = 0.f;
        if (c < L)
          x = !isV ? dWg[bht(bh, t0 + c, T, K) + col]
              : dd16 ? bf2f(reinterpret_cast<const bf16_t*>(dDl)[bht(bh, t0 + c, T, V) + col])
                     : dDl[bht(bh, t0 + c, T, V) + col];
        acc[r] = x;
      }
#pragma unroll 1
      for (int s = 16 * (I + 1); s < C; ++s) {
        const float xs = sX[s * XP + j];
        const float4* nrow = reinterpret_cast<const float4*>(sN + s * NS + 16 * I);
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const float4 nv = nrow[r4];
          acc[4 * r4 + 0] -= nv.x * xs;
          acc[4 * r4 + 1] -= nv.y * xs;
          acc[4 * r4 + 2] -= nv.z * xs;
          acc[4 * r4 + 3] -= nv.w * xs;
        }
      }
#pragma unroll
      for (int r = 14; r >= 0; --r) {
#pragma unroll
        for (int r2 = r + 1; r2 < 16; ++r2) acc[r] -= sN[(16 * I + r2) * NS + 16 * I + r] * acc[r2];
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int c = 16 * I + r;
        sX[c * XP + j] = acc[r];
        if (c < L) {
          if (isV) dv[bthk(b, t0 + c, h, col, T, H, V)] = f2bf(acc[r]);
          else dKg[bht(bh, t0 + c, T, K) + col] = acc[r];
        }
      }
    }
  }
  // stage [U | W] rows for dN
  stage_f32<C, V, XP>(U + bht(bh, t0, T, V), V, L, sUW);
  stage_f32<C, K, XP>(W + bht(bh, t0, T, K), K, L, sUW + V);
  __syncthreads();
  // dN = -(X [U|W]^T), strictly lower
  float* dNn = dNg + ((int64_t)bh * NT + n) * C * C;
  for (int tile = w; tile < 16; tile += 4) {
    const int I = tile >> 2, J = tile & 3;
    f32x4 acc = zero4();
    if (J <= I) {
      const int cA = 16 * I + (lane & 15), sB = 16 * J + (lane & 15);
#pragma unroll 8
      for (int st = 0; st < (V + K) / 4; ++st) {
        const int jj = 4 * st + (lane >> 4);
        acc = mfma4(sX[cA * XP + jj], sUW[sB * XP + jj], acc);
      }
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int c = 16 * I + 4 * (lane >> 4) + jj, s = 16 * J + (lane & 15);
      dNn[c * C + s] = (s < c) ? -acc[jj] : 0.f;
    }
  }
}

template <int K, int V, bool ISO>
__global__ __launch_bounds__(256) void mem_bwd_solve_exact_kernel(
    const bf16_t* __restrict__ k, const float* __restrict__ kap, const float* __restrict__ gc,
    const float* __restrict__ dDl, const float* __restrict__ dWg, const float* __restrict__ U,
    const float* __restrict__ W, int T, int H, int NT, int NB, const int* __restrict__ flags, bf16_t* __restrict__ dv,
    float* __restrict__ dKg, float* __restrict__ dNg, const float* __restrict__ k_rstd, bool dd16) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[ExactLds<K, V>::solve];
  if (!any_flagged(flags, NB)) return;
  for (int lin = blockIdx.x; lin < NB; lin += gridDim.x) {
    if (flags[lin] == 0) continue;
    __syncthreads();
    bwd_solve_exact_chunk<K, V, ISO>(k, kap, gc, dDl, dWg, U, W, T, H, NT, dv, dKg, dNg, lin % NT, lin / NT, k_rstd,
                                     dd16, lds);
  }
}

// ===========================================================================
// Backward, exact path for one chunk: gradients of q, k, kappa (beta) and g from dN, dM and
// the elementwise factors with per-block anchors and per-element diagonal blocks; runs only
// for the chunks the forward flagged.  Output tile (row block I, 16 channels); lane holds
// rows 16I + 4(lane/16) + j.
// ===========================================================================
template <int K, int V, bool ISO>
__device__ void bwd_contrib_exact_chunk(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const float* __restrict__ kap,
    const float* __restrict__ gc, const float* __restrict__ dNg, const float* __restrict__ dMg,
    const float* __restrict__ dQg, const float* __restrict__ dKg, const float* __restrict__ dKf,
    const float* __restrict__ dgl, int T, int H, int NT, float scale, bf16_t* __restrict__ dq,
    bf16_t* __restrict__ dk, float* __restrict__ dkap, float* __restrict__ dbeta, float* __restrict__ dg, int n,
    int bh, const float* __restrict__ q_rstd, const float* __restrict__ k_rstd, unsigned char* lds) {
  constexpr int KP = K + 4;
  constexpr int NCT = K / 16;  // channel tiles
  constexpr int KQ = QKStride<K, bf16_t>::value;
  static_assert(KQ == ExactLds<K, V>::KQ, "staged q / k stride");
  // lds: ExactLds::contrib bytes
  bf16_t* sQ = reinterpret_cast<bf16_t*>(lds);  // bf16 inputs are exact in bf16
  bf16_t* sK = sQ + C * KQ;
  float* sA = reinterpret_cast<float*>(sK + C * KQ);
  float* sG = sA + C * KP;
  float* sDN = sG + C * KP;
  float* sDM = sDN + C * NS;
  float* sSpan = sDM + C * NS;
  float* sColPart = sSpan + 4;          // per row block partial of sum_c dKf kappa e^{g_last - g}
  float* sDgLast = sColPart + 4 * K;    // dg of row L-1 before the g_last terms
  float* sBetaPart = sDgLast + K;       // iso: per (row, channel tile) partial of sum_i dkappa k
  const int b = bh / H, h = bh % H;
  const int t0 = n * C, L = min(C, T - t0);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  stage_chunk<K, ISO, bf16_t>(q, k, kap, gc, b, h, T, H, t0, L, sQ, sK, sA, sG, sSpan, q_rstd, k_rstd);
  stage_f32<C, C, NS>(dNg + ((int64_t)bh * NT + n) * C * C, C, C, sDN);
  stage_f32<C, C, NS>(dMg + ((int64_t)bh * NT + n) * C * C, C, C, sDM);
  for (int e = tid; e < 4 * K; e += 256) sColPart[e] = 0.f;
  __syncthreads();
  const int rowL = L - 1;
  for (int tile = w; tile < 4 * NCT; tile += 4) {
    const int I = tile / NCT, ct = tile % NCT;
    const int a = 16 * I;
    const bool fast = sSpan[I] <= kSpanMax;
    const int ich = 16 * ct + (lane & 15);  // this lane's output channel
    // ---- row-oriented: dk_N and dq_M (unscaled), anchor a ----
    f32x4 accK = zero4(), accQ = zero4();
    {
      const int cA = a + (lane & 15);
      const int nJ = fast ? I + 1 : I;
      for (int J = 0; J < nJ; ++J) {
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const int s = 16 * J + 4 * st + (lane >> 4);
          const float br = sA[s * KP + ich] * exp2f(sG[a * KP + ich] - sG[s * KP + ich]);
          accK = mfma4(sDN[cA * NS + s], br, accK);
          accQ = mfma4(sDM[cA * NS + s], br, accQ);
        }
      }
    }
    // ---- column-oriented: dkappa_N, dkappa_M ----
    f32x4 accK2 = zero4(), accQ2 = zero4(), accK2d = zero4(), accQ2d = zero4();
    {
      const int sA_ = a + (lane & 15);  // output row (as source index s)
      if (I < 3) {
        const int bnc = 16 * (I + 1);
        for (int Ip = I + 1; Ip < 4; ++Ip) {
#pragma unroll
          for (int st = 0; st < 4; ++st) {
            const int c = 16 * Ip + 4 * st + (lane >> 4);
            const float f = exp2f(sG[c * KP + ich] - sG[bnc * KP + ich]);
            accK2 = mfma4(sDN[c * NS + sA_], lds_f(sK, c * KQ + ich) * f, accK2);
            accQ2 = mfma4(sDM[c * NS + sA_], lds_f(sQ, c * KQ + ich) * f, accQ2);
          }
        }
      }
      if (fast) {
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const int c = a + 4 * st + (lane >> 4);
          const float f = exp2f(sG[c * KP + ich] - sG[a * KP + ich]);
          accK2d = mfma4(sDN[c * NS + sA_], lds_f(sK, c * KQ + ich) * f, accK2d);
          accQ2d = mfma4(sDM[c * NS + sA_], lds_f(sQ, c * KQ + ich) * f, accQ2d);
        }
      }
    }
    // ---- assemble ----
    const int bnc = I < 3 ? 16 * (I + 1) : a;
    const float ga = sG[a * KP + ich], gb = sG[bnc * KP + ich], glast = sG[rowL * KP + ich];
    float colpart = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = a + 4 * (lane >> 4) + j;
      const float gcv = sG[c * KP + ich];
      const float kc = lds_f(sK, c * KQ + ich), qc = lds_f(sQ, c * KQ + ich), ac = sA[c * KP + ich];
      float dkN, dqM, dkapN, dkapM;
      if (fast) {
        const float el = exp2f(gcv - ga);
        dkN = accK[j] * el;
        dqM = accQ[j] * el;
        const float er = exp2f(ga - gcv);
        dkapN = accK2[j] * exp2f(gb - gcv) + accK2d[j] * er;
        dkapM = accQ2[j] * exp2f(gb - gcv) + accQ2d[j] * er;
      } else {
        const float el = exp2f(gcv - ga);
        dkN = accK[j] * el;
        dqM = accQ[j] * el;
        dkapN = I < 3 ? accK2[j] * exp2f(gb - gcv) : 0.f;
        dkapM = I < 3 ? accQ2[j] * exp2f(gb - gcv) : 0.f;
        // exact diagonal block
        for (int s = a; s < a + 16; ++s) {
          const float gs = sG[s * KP + ich];
          if (s <= c) {
            const float e = exp2f(gcv - gs) * sA[s * KP + ich];
            if (s < c) dkN += sDN[c * NS + s] * e;
            dqM += sDM[c * NS + s] * e;
          }
          if (s >= c) {
            const float e = exp2f(gs - gcv);
            if (s > c) dkapN += sDN[s * NS + c] * lds_f(sK, s * KQ + ich) * e;
            dkapM += sDM[s * NS + c] * lds_f(sQ, s * KQ + ich) * e;
          }
        }
      }
      dqM *= scale;
      dkapM *= scale;
      float dkv = dkN, dqv = dqM, dav = dkapN + dkapM, dgv = 0.f;
      if (c < L) {
        const int64_t o = bht(bh, t0 + c, T, K) + ich;
        const float ec = exp2f(gcv);
        const float f = exp2f(glast - gcv);
        const float dkg = dKg[o], dqg = dQg[o], dkf = dKf[o];
        dkv += dkg * ec;
        dqv += scale * dqg * ec;
        dav += dkf * f;
        dgv = dkg * kc * ec + dqg * scale * qc * ec - dkf * ac * f;
        colpart += dkf * ac * f;
        dgv += kc * dkN - ac * dkapN + qc * dqM - ac * dkapM;
      }
      if (c < L) {
        if (ISO) {
          // kappa = beta k:  dk += beta dkappa;  dbeta = sum_i dkappa_i k_i (reduced below).
          // Lanes sharing (lane >> 4) hold the same row, so the 16-lane reduction stays in one branch.
          const float bc = kap[((int64_t)b * T + t0 + c) * H + h];
          dkv += bc * dav;
          float part = dav * kc;
          // reduce over the 16 channels of this tile (lanes sharing lane>>4)
#pragma unroll
          for (int o2 = 1; o2 < 16; o2 <<= 1) part += __shfl_xor(part, o2, 64);
          if ((lane & 15) == 0) sBetaPart[c * NCT + ct] = part;
        } else {
          dkap[bthk(b, t0 + c, h, ich, T, H, K)] = dav;
        }
        dq[bthk(b, t0 + c, h, ich, T, H, K)] = f2bf(dqv);
        dk[bthk(b, t0 + c, h, ich, T, H, K)] = f2bf(dkv);
        if (c == rowL) sDgLast[ich] = dgv;
        else dg[bthk(b, t0 + c, h, ich, T, H, K)] = dgv;
      }
    }
    // column partial of the g_last term over this lane's 4 rows, then over the 4 row groups
    colpart += __shfl_xor(colpart, 16, 64);
    colpart += __shfl_xor(colpart, 32, 64);
    if (lane < 16) sColPart[I * K + ich] = colpart;
  }
  __syncthreads();
  if (tid < K) {
    const int i = tid;
    const float extra = dgl[((int64_t)bh * NT + n) * K + i] + sColPart[i] + sColPart[K + i] + sColPart[2 * K + i] +
                        sColPart[3 * K + i];
    dg[bthk(b, t0 + rowL, h, i, T, H, K)] = sDgLast[i] + extra;
  }
  if (ISO && tid < L) {
    float s = 0.f;
    for (int ct = 0; ct < NCT; ++ct) s += sBetaPart[tid * NCT + ct];
    dbeta[((int64_t)b * T + t0 + tid) * H + h] = s;
  }
}

template <int K, int V, bool ISO>
__global__ __launch_bounds__(256) void mem_bwd_contrib_exact_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const float* __restrict__ kap,
    const float* __restrict__ gc, const float* __restrict__ dNg, const float* __restrict__ dMg,
    const float* __restrict__ dQg, const float* __restrict__ dKg, const float* __restrict__ dKf,
    const float* __restrict__ dgl, int T, int H, int NT, int NB, const int* __restrict__ flags, float scale,
    bf16_t* __restrict__ dq, bf16_t* __restrict__ dk, float* __restrict__ dkap, float* __restrict__ dbeta,
    float* __restrict__ dg, const float* __restrict__ q_rstd, const float* __restrict__ k_rstd) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[ExactLds<K, V>::contrib];
  if (!any_flagged(flags, NB)) return;
  for (int lin = blockIdx.x; lin < NB; lin += gridDim.x) {
    if (flags[lin] == 0) continue;
    __syncthreads();
    bwd_contrib_exact_chunk<K, V, ISO>(q, k, kap, gc, dNg, dMg, dQg, dKg, dKf, dgl, T, H, NT, scale, dq, dk, dkap,
                                       dbeta, dg, lin % NT, lin / NT, q_rstd, k_rstd, lds);
  }
}

// The in-op L2 norm's backward for the rows of the flagged chunks (whose dq, dk the exact kernel
// above wrote for the normalised operands y = bf16(x rstd) of the raw q, k): dx = rstd (dy - y (y . dy)),
// in place.
// One wave per row (K / 64 elements per lane); a row is read whole before it is written.
template <int K>
__device__ void l2norm_bwd_chunk_rows(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
                                      const float* __restrict__ q_rstd, const float* __restrict__ k_rstd, int T,
                                      int H, int n, int bh, bf16_t* __restrict__ dq, bf16_t* __restrict__ dk) {
  constexpr int PL = K / 64;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  {
    const int b = bh / H, h = bh % H;
    const int t0 = n * C, L = min(C, T - t0);
    for (int r = w; r < 2 * L; r += 4) {
      const bool isq = r < L;
      const int c = isq ? r : r - L;
      const int64_t row = ((int64_t)b * T + t0 + c) * H + h;
      const bf16_t* x = isq ? q : k;
      bf16_t* d = isq ? dq : dk;
      const float rs = (isq ? q_rstd : k_rstd)[row];
      float y[PL], g[PL], dot = 0.f;
#pragma unroll
      for (int j = 0; j < PL; ++j) {
        y[j] = l2n(bf2f(x[row * K + lane + 64 * j]), rs);
        g[j] = bf2f(d[row * K + lane + 64 * j]);
        dot += y[j] * g[j];
      }
      dot = wave_sum(dot);
#pragma unroll
      for (int j = 0; j < PL; ++j) d[row * K + lane + 64 * j] = f2bf(rs * (g[j] - y[j] * dot));
    }
  }
}
template <int K>
__global__ __launch_bounds__(256) void l2norm_bwd_flagged_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const float* __restrict__ q_rstd,
    const float* __restrict__ k_rstd, int T, int H, int NT, int NB, const int* __restrict__ flags,
    bf16_t* __restrict__ dq, bf16_t* __restrict__ dk) {
  if (!any_flagged(flags, NB)) return;
  for (int lin = blockIdx.x; lin < NB; lin += gridDim.x)
    if (flags[lin] != 0) l2norm_bwd_chunk_rows<K>(q, k, q_rstd, k_rstd, T, H, lin % NT, lin / NT, dq, dk);
}

// The whole exact backward of each flagged chunk in one workgroup: the solves (dv, dKg, dN), then the
// gradients from them, then (in-op norm) the norm's backward of its q, k rows.  Each step reads only what
// the previous ones wrote for the same chunk; the barrier between steps orders those global writes before
// the next step's reads (the workgroup's waves share one CU's caches), and the steps' LDS arrays share one
// pool.  One launch instead of the two or three a call with both exact stages would make.
template <int K, int V, bool ISO>
__global__ __launch_bounds__(256) void mem_bwd_exact_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const float* __restrict__ kap,
    const float* __restrict__ gc, const float* __restrict__ dDl, const float* __restrict__ dWg,
    const float* __restrict__ U, const float* __restrict__ W, const float* __restrict__ dMg,
    const float* __restrict__ dQg, const float* __restrict__ dKf, const float* __restrict__ dgl, int T, int H, int NT,
    int NB, const int* __restrict__ flags, float scale, bf16_t* __restrict__ dv, float* __restrict__ dKg,
    float* __restrict__ dNg, bf16_t* __restrict__ dq, bf16_t* __restrict__ dk, float* __restrict__ dkap,
    float* __restrict__ dbeta, float* __restrict__ dg, const float* __restrict__ q_rstd,
    const float* __restrict__ k_rstd, bool dd16) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[ExactLds<K, V>::both];
  if (!any_flagged(flags, NB)) return;
  for (int lin = blockIdx.x; lin < NB; lin += gridDim.x) {
    if (flags[lin] == 0) continue;
    const int n = lin % NT, bh = lin / NT;
    __syncthreads();
    bwd_solve_exact_chunk<K, V, ISO>(k, kap, gc, dDl, dWg, U, W, T, H, NT, dv, dKg, dNg, n, bh, k_rstd, dd16, lds);
    __syncthreads();
    bwd_contrib_exact_chunk<K, V, ISO>(q, k, kap, gc, dNg, dMg, dQg, dKg, dKf, dgl, T, H, NT, scale, dq, dk, dkap,
                                       dbeta, dg, n, bh, q_rstd, k_rstd, lds);
    if (q_rstd) {
      __syncthreads();
      l2norm_bwd_chunk_rows<K>(q, k, q_rstd, k_rstd, T, H, n, bh, dq, dk);
    }
  }
}

inline int cdiv(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

// Chunk groups of the serial state passes (kdn_state.h, GroupPlan).  With few B*H*V/64 workgroups a
// two-level scan fills the chip.  Cost model in chunk steps, fitted to measured passes (both the
// forward pass, two workgroups per CU, and the reverse pass, one): a launch of n workgroups costs
// max(1, n / 256) times its groups' m steps; pass A runs the first group (V/64 slices per head) and
// the NG - 2 middle groups' maps ((V + K)/64 slices), pass C the NG - 1 later groups, pass B NG - 2
// combine steps.  Once the single pass occupies half the CUs, per-step contention makes the extra
// map work a loss (B4 H18: one pass 334 us, three groups 441 us), so NG = 1 there.
// Measured optima: B1 H18 T4096 -> 8 groups (forward 272 -> 144 us, reverse 418 -> 225 us),
// B2 -> 4, B1 T32768 -> 8 (forward 2163 -> 879 us).
constexpr int kStateSlots = 256;
struct GroupCount {
  int NG, m;
};
inline GroupCount plan_groups(int BH, int NT, int K, int V) {
  const int NV = V / kdn_state::state_cols(V), NPHI = K / kdn_state::state_cols(V);
  GroupCount best{1, NT};
  if ((int64_t)BH * NV > kStateSlots / 2) return best;
  auto load = [](int64_t n) { return n > kStateSlots ? (double)n / kStateSlots : 1.0; };
  double best_cost = NT;
  for (int NG = 2; NG <= 64 && 2 * NG <= NT; ++NG) {
    const int m = cdiv(NT, NG);
    if ((int64_t)(NG - 1) * m >= NT) continue;  // the last group would be empty
    const int64_t a = (int64_t)BH * NV + (int64_t)BH * (NG - 2) * (NV + NPHI);
    const int64_t c = (int64_t)BH * (NG - 1) * NV;
    const double cost = (load(a) + load(c)) * m + (NG - 2);
    if (cost < best_cost) {
      best_cost = cost;
      best = GroupCount{NG, m};
    }
  }
  return best;
}
// floats of a grouped pass's buffers: Sg [BH][NG][K][V] and Mg [BH][NG][K][V + K]
inline int64_t group_floats(int64_t BH, GroupCount gc, int K, int V) {
  return gc.NG > 1 ? BH * gc.NG * K * (2 * (int64_t)V + K) : 0;
}
inline int64_t round64(int64_t x) { return (x + 63) / 64 * 64; }

// Precision of the per-chunk copies only the backward reads (the forward pass's h and delta, the
// reverse pass's dh and d delta; kdn_state::HB_* bits, set = bf16).  The isotropic scan stores h and dh
// in bf16 (its reference's backward keeps all four in the input dtype: FLA's chunk_gated_delta_rule
// allocates h, v_new, dh and dv2 like k): half the bytes of the two largest copies, written by the
// state passes and read by the chunk backward, whose products with them take one or two bf16 MFMAs
// instead of three.  delta and d delta stay fp32: in bf16 they moved the parameter gradients that sum
// over every token with heavy cancellation (dA_log, the omega / r biases) by up to 1e-2 of their size
// at B4 T4096 H18, against 4e-4 with bf16 h and dh alone.  The diagonal scan keeps fp32 (its reference
// kernel keeps an fp32 h), and so does a scan whose state passes run in chunk groups (few B*H streams),
// whose first group's chunk-parallel readout reads the forward's h and delta.  The recurrences
// themselves and every output stay as before; the forward and the backward take the same decision from
// the shape.
constexpr int kIsoHalfCopies = kdn_state::HB_H | kdn_state::HB_DH;
inline int half_copies(int iso, GroupCount gc) { return iso && gc.NG == 1 ? kIsoHalfCopies : 0; }
// Calls f with the copies' precision mask as a compile-time constant.
template <typename F>
inline void with_copy_mask(int hm, F f) {
  if (hm == kIsoHalfCopies) f(std::integral_constant<int, kIsoHalfCopies>{});
  else f(std::integral_constant<int, 0>{});
}

// saved-buffer layout (floats), TT = B*H*T, NB = B*H*NT
struct MemLayout {
  int64_t U, W, Kf, Qg, M, A, h, D, flags, grp, mid, total;
  GroupCount gc;
  MemLayout(int B, int T, int H, int K, int V) {
    const int64_t TT = (int64_t)B * H * T, NB = (int64_t)B * H * cdiv(T, C);
    gc = plan_groups(B * H, cdiv(T, C), K, V);
    U = 0;
    W = U + TT * V;
    Kf = W + TT * K;
    Qg = Kf + TT * K;
    M = Qg + TT * K;
    A = M + NB * C * C;
    h = A + NB * C * C;
    D = h + NB * K * V;
    flags = D + TT * V;  // NB ints: chunk taken by the exact intra-chunk path
    grp = round64(flags + NB);  // the forward state pass's group buffers (dead after the forward)
    mid = grp + group_floats((int64_t)B * H, gc, K, V);  // the overlapped forward's carried state
    total = mid + (int64_t)B * H * K * V;
  }
};
struct BwdLayout {
  int64_t dh, dD, dQg, dW, dKf, dM, dgl, dKg, dN, carry, grp, total;
  GroupCount gc;
  BwdLayout(int B, int T, int H, int K, int V) {
    const int64_t TT = (int64_t)B * H * T, NB = (int64_t)B * H * cdiv(T, C);
    gc = plan_groups(B * H, cdiv(T, C), K, V);
    dh = 0;
    dD = dh + NB * K * V;
    dQg = dD + TT * V;
    dW = dQg + TT * K;
    dKf = dW + TT * K;
    dM = dKf + TT * K;
    dgl = dM + NB * C * C;
    dKg = dgl + NB * K;
    dN = dKg + TT * K;
    carry = round64(dN + NB * C * C);  // two cotangents carried between segments of the reverse pass
    grp = carry + 2 * (int64_t)B * H * K * V;  // the reverse state pass's group buffers
    total = grp + group_floats((int64_t)B * H, gc, K, V);
  }
};

// Overlapped schedule of the reverse state pass and the chunk backward (one call with both).  With
// one chunk group the pass occupies B*H*V/64 workgroups, one per CU (144 at B4 H18), and leaves
// `idle` CUs.  It runs in two segments: the last m1 chunks, then the rest (the state gradient
// crosses the boundary in fp32, so results are bit-identical to one pass).  Once the first segment
// is done, a second stream runs the chunk-backward tasks of its chunks: the second segment's
// workgroups take the CUs the first one frees (the side launch starts a few microseconds later), and
// the side launch's workgroups fill the idle CUs and backfill them as they finish.  The remaining
// tasks run at full width after the pass.  A chunk-backward task lasts about kStepsPerTask chunk
// steps of the pass running beside it (~36 us against ~5.7 us), which sizes the first segment so
// that its tasks keep the idle CUs busy until the pass ends.
constexpr float kStepsPerTask = 6.4f;
constexpr unsigned kSideDelayTicks = 300;  // of the 100 MHz wall clock: 3 us
struct BwdOverlap {
  int m1 = 0, side_tasks = 0;
};
inline BwdOverlap plan_bwd_overlap(int BH, int NT, int NV, GroupCount gc, int cus) {
  BwdOverlap o;
  const int idle = cus - BH * NV;
  if (gc.NG != 1 || idle < 32 || NT < 16) return o;
  const int m1 = max(1, min(NT / 2, (int)ceilf((float)NT * idle / (kStepsPerTask * BH + idle))));
  const int iters = (int)lrintf((NT - m1) / kStepsPerTask);
  o.m1 = m1;
  o.side_tasks = min(m1 * BH, iters * idle);
  return o;
}
// Overlapped schedule of the forward (one call with the intra-chunk build and the state pass): the build
// of the first m1 chunks, then their state pass beside the build of the rest on a second stream, then
// the rest's pass (see mem_fwd_impl).  The pass holds B*H*V/64 CUs; the side build's workgroups (three
// per CU, each lasting about kBuildSteps chunk steps of the pass: the diagonal build is ~15% longer) take
// the `idle` ones, so m1 balances the first range's pass against the second range's build there.
// Measured at B4 T4096 H18 (m1 swept 30 .. 45): best at 39 (isotropic) and 42 (diagonal).
constexpr float kBuildStepsIso = 7.3f, kBuildStepsDiag = 9.0f;
inline int plan_fwd_overlap(int BH, int NT, int NV, int cus, bool iso) {
  const int idle = cus - BH * NV;
  if (idle < 32 || NT < 8) return 0;
  const float r = BH * (iso ? kBuildStepsIso : kBuildStepsDiag) / (3.f * idle);
  return max(1, min(NT - 1, (int)lrintf(NT * r / (1.f + r))));
}

// One wave that returns after `ticks` of the constant 100 MHz clock (bounded wait, no memory access).
__global__ void side_delay_kernel(unsigned ticks) {
  const uint64_t t0 = wall_clock64();
  while (wall_clock64() - t0 < ticks) __builtin_amdgcn_s_sleep(8);
}

// The second stream of a device and the events that order it against the caller's stream: made
// on first use (default priority, non-blocking), kept until the process ends.  Every call on a
// device shares them, so one schedule's enqueue holds the mutex.
struct SideQueue {
  hipStream_t s = nullptr;
  hipEvent_t ev[2] = {};
  int cus = 0;  // compute units of the device
};
std::mutex g_side_mu;
constexpr int kMaxDevices = 64;
SideQueue g_side[kMaxDevices];
// Call with g_side_mu held.
int side_queue(SideQueue** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return KDN_ERR_ARG;
  SideQueue& q = g_side[dev];
  if (!q.s) {
    if ((e = hipDeviceGetAttribute(&q.cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return (int)e;
    for (auto& ev : q.ev)
      if (!ev && (e = hipEventCreateWithFlags(&ev, hipEventDisableTiming)) != hipSuccess) return (int)e;
    if ((e = hipStreamCreateWithFlags(&q.s, hipStreamNonBlocking)) != hipSuccess) {
      q.s = nullptr;
      return (int)e;
    }
  }
  *out = &q;
  return 0;
}
// true once this device's side queue exists
inline bool side_ready() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
  std::lock_guard<std::mutex> lock(g_side_mu);
  return g_side[dev].s != nullptr;
}
// `to` waits for the work enqueued on `from` so far
inline int stream_wait(hipStream_t to, hipStream_t from, hipEvent_t ev) {
  hipError_t e = hipEventRecord(ev, from);
  if (e == hipSuccess) e = hipStreamWaitEvent(to, ev, 0);
  return (int)e;
}

// Launch pass A / B / C of a state pass (or the single serial pass).  launch(grid, plan) issues the
// state kernel of one pass.
template <int K, int V, typename Launch>
int run_state_pass(int BH, GroupCount gc, float* grp, bool reverse, hipStream_t stream, Launch launch) {
  constexpr int NV = V / kdn_state::state_cols(V), NS = NV + K / kdn_state::state_cols(V);
  kdn_state::GroupPlan P{gc.NG, gc.m, 0, grp, grp + (gc.NG > 1 ? (int64_t)BH * gc.NG * K * V : 0)};
  if (gc.NG == 1) {
    launch(dim3(BH * NV), P);
    KDN_CHECK_LAUNCH();
    return 0;
  }
  launch(dim3(BH * (gc.NG - 1) * NS), P);  // pass A
  KDN_CHECK_LAUNCH();
  if (gc.NG > 2) {  // pass B
    if (reverse)
      hipLaunchKernelGGL((kdn_state::state_combine_kernel<K, V>), dim3(BH * NV), dim3(kdn_state::state_threads(V)), 0,
                         stream, P, BH, gc.NG - 2, gc.NG - 2, -1);
    else
      hipLaunchKernelGGL((kdn_state::state_combine_kernel<K, V>), dim3(BH * NV), dim3(kdn_state::state_threads(V)), 0,
                         stream, P, BH, 1, gc.NG - 2, 1);
    KDN_CHECK_LAUNCH();
  }
  P.pass = 1;
  launch(dim3(BH * (gc.NG - 1) * NV), P);  // pass C
  KDN_CHECK_LAUNCH();
  return 0;
}


template <int K, int V>
int mem_fwd_impl(const bf16_t* q, const bf16_t* k, const float* kap, int iso, const bf16_t* v, const float* gc, int B,
                 int T, int H, float scale, const float* h0, float* saved, float* ht, void* o, int o_bf16,
                 float* q_rstd, float* k_rstd, int stages, hipStream_t stream) {
  const int NT = cdiv(T, C);
  MemLayout lay(B, T, H, K, V);
  float *U = saved + lay.U, *W = saved + lay.W, *Kf = saved + lay.Kf, *Qg = saved + lay.Qg, *M = saved + lay.M,
        *A = saved + lay.A, *hb = saved + lay.h, *D = saved + lay.D;
  int* flags = reinterpret_cast<int*>(saved + lay.flags);
  const int hm = half_copies(iso, lay.gc);
  // bit 3 (stages >= 0): no backward follows, so A^T and, where the readout is fused, h and delta
  // are not written
  const bool infer = stages >= 0 && (stages & 8) != 0;
  float* Asave = infer ? nullptr : A;
  // the intra-chunk build of chunks n0 .. n1 - 1 on stream s: the single-anchor kernel, then one launch for the
  // chunks it flagged (the block-anchor path, and the exact path for those it leaves flagged)
  auto launch_intra = [&](int n0, int n1, hipStream_t s) {
    const dim3 gchunk(n1 - n0, B * H);
    const int gx = min(B * H * (n1 - n0), 256);  // one workgroup per CU fits (its LDS)
    // the in-op L2 norm (q_rstd given) is a template variant: its row loads would otherwise cost the
    // plain kernels registers
#define KDN_INTRA(ISO_, NORM_)                                                                                         \
  do {                                                                                                                 \
    hipLaunchKernelGGL((kdn_intra::intra_fwd_kernel<K, V, ISO_, NORM_>), gchunk, dim3(256), 0, s, q, k, kap, v, gc, T, \
                       H, NT, scale, U, W, Kf, Qg, M, Asave, flags, q_rstd, k_rstd, n0);                               \
    hipLaunchKernelGGL((intra_fwd_flagged_kernel<K, V, ISO_, NORM_>), dim3(gx), dim3(256), 0, s, q, k, kap, v, gc, T,  \
                       H, NT, B * H, n0, n1, scale, U, W, Kf, Qg, M, Asave, flags, q_rstd, k_rstd);                  \
  } while (0)
    if (iso && q_rstd) KDN_INTRA(true, true);
    else if (iso) KDN_INTRA(true, false);
    else if (q_rstd) KDN_INTRA(false, true);
    else KDN_INTRA(false, false);
#undef KDN_INTRA
  };
  auto launch_ro = [&](dim3 grid, const kdn_state::GroupPlan& P, float* hstore, float* dstore, int mask,
                       const float* hin, float* hout) {
    const dim3 bs(2 * kdn_state::state_threads(V));
    with_copy_mask(mask, [&](auto hmc) {
      constexpr int HM = decltype(hmc)::value;
      if (o_bf16)
        hipLaunchKernelGGL((kdn_state::state_fwd_kernel<K, V, bf16_t, true, HM>), grid, bs, 0, stream, U, W, Kf, gc,
                           hin, T, H, NT, B * H, hstore, dstore, hout, P, Qg, M, (bf16_t*)o);
      else
        hipLaunchKernelGGL((kdn_state::state_fwd_kernel<K, V, float, true, HM>), grid, bs, 0, stream, U, W, Kf, gc,
                           hin, T, H, NT, B * H, hstore, dstore, hout, P, Qg, M, (float*)o);
    });
  };
  // Overlapped schedule (bits 0, 1 and 2 in one call, one chunk group): the state pass (with the readout
  // fused) occupies B*H*V/64 CUs, one workgroup each, and leaves the rest idle.  The sequence runs in two
  // chunk ranges: the build of the first m1 chunks, then that range's state pass on `stream` while the
  // second range's build runs on the side stream, then the second range's pass from the carried state
  // (saved + mid, fp32: the same state the single pass holds, so every output is bit-identical).
  if ((stages & 7) == 7 && lay.gc.NG == 1) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) != hipSuccess) return KDN_ERR_ARG;
    if (cap == hipStreamCaptureStatusNone || side_ready()) {
      std::lock_guard<std::mutex> lock(g_side_mu);
      SideQueue* sq = nullptr;
      int rc = side_queue(&sq);
      if (rc) return rc;
      const int m1 = plan_fwd_overlap(B * H, NT, V / kdn_state::state_cols(V), sq->cus, iso != 0);
      if (m1 > 0) {
        const dim3 grid(B * H * (V / kdn_state::state_cols(V)));
        float* mid = saved + lay.mid;
        launch_intra(0, m1, stream);
        KDN_CHECK_LAUNCH();
        if ((rc = stream_wait(sq->s, stream, sq->ev[0]))) return rc;
        launch_intra(m1, NT, sq->s);
        KDN_CHECK_LAUNCH();
        launch_ro(grid, kdn_state::GroupPlan{1, NT, 0, nullptr, nullptr, 0, m1}, infer ? nullptr : hb,
                  infer ? nullptr : D, hm, h0, mid);
        KDN_CHECK_LAUNCH();
        if ((rc = stream_wait(stream, sq->s, sq->ev[1]))) return rc;
        launch_ro(grid, kdn_state::GroupPlan{1, NT, 0, nullptr, nullptr, m1, NT}, infer ? nullptr : hb,
                  infer ? nullptr : D, hm, mid, ht);
        KDN_CHECK_LAUNCH();
        return 0;
      }
    }
  }
  if (stages & 1) {
    launch_intra(0, NT, stream);
    KDN_CHECK_LAUNCH();
  }
  auto launch_readout = [&](int NR) {  // chunk-parallel readout O = Qg h + M delta of the first NR chunks
    const int NCH = NR * B * H;        // chunk-heads; with two V halves the grid is padded to pairs of 8
    const dim3 gr(V / 64 == 2 ? 16 * cdiv(NCH, 8) : NCH);
    with_copy_mask(hm, [&](auto hmc) {
      constexpr int HM = decltype(hmc)::value;
      if (o_bf16)
        hipLaunchKernelGGL((kdn_state::readout_kernel<K, V, bf16_t, HM>), gr, dim3(256), 0, stream, Qg, M, hb, D, T, H,
                           NT, NR, B * H, (bf16_t*)o);
      else
        hipLaunchKernelGGL((kdn_state::readout_kernel<K, V, float, HM>), gr, dim3(256), 0, stream, Qg, M, hb, D, T, H,
                           NT, NR, B * H, (float*)o);
    });
  };
  if ((stages & 6) == 6) {  // state pass with the readout fused
    const GroupCount gcnt = lay.gc;
    if (gcnt.NG == 1) {
      launch_ro(dim3(B * H * (V / kdn_state::state_cols(V))), kdn_state::GroupPlan{1, NT, 0, nullptr, nullptr},
                infer ? nullptr : hb, infer ? nullptr : D, hm, h0, ht);
      KDN_CHECK_LAUNCH();
      return 0;
    }
    // two-level: pass A (first group, which stores its h and delta, and the middle groups' maps),
    // the combine, pass C with the readout fused, then the first group's readout
    constexpr int NV = V / kdn_state::state_cols(V), NS = NV + K / kdn_state::state_cols(V);
    float* grp = saved + lay.grp;
    kdn_state::GroupPlan P{gcnt.NG, gcnt.m, 0, grp, grp + (int64_t)B * H * gcnt.NG * K * V};
    hipLaunchKernelGGL((kdn_state::state_fwd_kernel<K, V>), dim3(B * H * (gcnt.NG - 1) * NS),
                       dim3(kdn_state::state_threads(V)), 0, stream, U, W, Kf, gc, h0, T, H, NT, B * H, hb, D, ht, P);
    KDN_CHECK_LAUNCH();
    if (gcnt.NG > 2) {
      hipLaunchKernelGGL((kdn_state::state_combine_kernel<K, V>), dim3(B * H * NV), dim3(kdn_state::state_threads(V)),
                         0, stream, P, B * H, 1, gcnt.NG - 2, 1);
      KDN_CHECK_LAUNCH();
    }
    P.pass = 1;
    launch_ro(dim3(B * H * (gcnt.NG - 1) * NV), P, infer ? nullptr : hb, infer ? nullptr : D, 0, h0, ht);
    KDN_CHECK_LAUNCH();
    launch_readout(gcnt.m);
    KDN_CHECK_LAUNCH();
    return 0;
  }
  if (stages & 2) {  // serial state pass (one- or two-level): h per chunk, delta, final state
    const dim3 bs(kdn_state::state_threads(V));
    const int rc = run_state_pass<K, V>(
        B * H, lay.gc, saved + lay.grp, false, stream, [&](dim3 grid, const kdn_state::GroupPlan& P) {
          with_copy_mask(hm, [&](auto hmc) {
            hipLaunchKernelGGL((kdn_state::state_fwd_kernel<K, V, float, false, decltype(hmc)::value>), grid, bs, 0,
                               stream, U, W, Kf, gc, h0, T, H, NT, B * H, hb, D, ht, P);
          });
        });
    if (rc) return rc;
  }
  if (stages & 4) {  // chunk-parallel readout O = Qg h + M delta of every chunk
    launch_readout(NT);
    KDN_CHECK_LAUNCH();
  }
  return 0;
}

template <int K, int V, typename TDO>
int mem_bwd_impl(const bf16_t* q, const bf16_t* k, const float* kap, int iso, const float* gc, int B, int T, int H,
                 float scale, const TDO* dO, const float* dht, const float* saved, float* work, bf16_t* dq,
                 bf16_t* dk, float* dkap, float* dbeta, bf16_t* dv, float* dg, float* dh0, const float* q_rstd,
                 const float* k_rstd, int stages, hipStream_t stream) {
  const int NT = cdiv(T, C);
  MemLayout lay(B, T, H, K, V);
  BwdLayout bl(B, T, H, K, V);
  const float *U = saved + lay.U, *W = saved + lay.W, *Kf = saved + lay.Kf, *Qg = saved + lay.Qg,
              *M = saved + lay.M, *A = saved + lay.A, *hb = saved + lay.h, *D = saved + lay.D;
  const int* flags = reinterpret_cast<const int*>(saved + lay.flags);
  float *dh = work + bl.dh, *dD = work + bl.dD, *dQg = work + bl.dQg, *dW = work + bl.dW, *dKf = work + bl.dKf,
        *dM = work + bl.dM, *dgl = work + bl.dgl, *dKg = work + bl.dKg, *dN = work + bl.dN;
  const int hm = half_copies(iso, bl.gc);
  constexpr int NV = V / kdn_state::state_cols(V);
  const dim3 bs(2 * kdn_state::state_threads(V));  // helper waves take M^T dO and Qg^T dO off the chain
  auto launch_state = [&](dim3 grid, const kdn_state::GroupPlan& P, const float* dS_in, float* dS_out,
                          hipStream_t st) {
    with_copy_mask(hm, [&](auto hmc) {
      hipLaunchKernelGGL((kdn_state::state_bwd_kernel<K, V, TDO, true, decltype(hmc)::value>), grid, bs, 0, st, M, Kf,
                         Qg, W, gc, dO, dS_in, T, H, NT, B * H, dh, dD, dS_out, P);
    });
  };
  // every chunk's products with h / dh; the solves and gradients of the unflagged ones: the
  // chunk-head tasks task0 .. task_end - 1 (order of chunk_bwd_task: last chunks first)
  auto launch_chunk = [&](int task0, int task_end, hipStream_t st) {
#define KDN_CHUNK_BWD(ISO_, HB_)                                                                                    \
  hipLaunchKernelGGL((kdn_bwd::chunk_bwd_kernel<K, V, ISO_, TDO, HB_>), dim3(task_end - task0), dim3(512), 0, st, hb, \
                     dh, D, dD, dO, A, U, W, flags, q, k, kap, gc, q_rstd, k_rstd, T, H, NT, B * H, task0, scale, dv, \
                     dq, dk, dkap, dbeta, dg, dQg, dW, dKf, dM, dgl)
    if (iso && hm == kIsoHalfCopies) KDN_CHUNK_BWD(true, kIsoHalfCopies);
    else if (iso) KDN_CHUNK_BWD(true, 0);
    else KDN_CHUNK_BWD(false, 0);
#undef KDN_CHUNK_BWD
  };
  const int tasks = NT * B * H;
  bool overlapped = false;
  // a stream under graph capture takes the overlapped schedule only once the side queue exists (it
  // is made outside capture: stream and event creation are not capturable)
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cap) != hipSuccess) return KDN_ERR_ARG;
  if ((stages & 3) == 3 && bl.gc.NG == 1 && (cap == hipStreamCaptureStatusNone || side_ready())) {
    std::lock_guard<std::mutex> lock(g_side_mu);
    SideQueue* sq = nullptr;
    int rc = side_queue(&sq);
    if (rc) return rc;
    const BwdOverlap ov = plan_bwd_overlap(B * H, NT, NV, bl.gc, sq->cus);
    if (ov.side_tasks > 0) {
      const int c1 = NT - ov.m1;
      float* carry = work + bl.carry;
      launch_state(dim3(B * H * NV), kdn_state::GroupPlan{1, NT, 0, nullptr, nullptr, c1, NT}, dht, carry, stream);
      KDN_CHECK_LAUNCH();
      if ((rc = stream_wait(sq->s, stream, sq->ev[0]))) return rc;
      // a few microseconds on the side stream first, so that the second segment's workgroups are
      // dispatched onto the CUs the first one frees before the side launch competes for them
      hipLaunchKernelGGL(side_delay_kernel, dim3(1), dim3(64), 0, sq->s, kSideDelayTicks);
      KDN_CHECK_LAUNCH();
      launch_chunk(0, ov.side_tasks, sq->s);
      KDN_CHECK_LAUNCH();
      launch_state(dim3(B * H * NV), kdn_state::GroupPlan{1, NT, 0, nullptr, nullptr, 0, c1}, carry, dh0, stream);
      KDN_CHECK_LAUNCH();
      launch_chunk(ov.side_tasks, tasks, stream);
      KDN_CHECK_LAUNCH();
      if ((rc = stream_wait(stream, sq->s, sq->ev[1]))) return rc;
      overlapped = true;
    }
  }
  if (!overlapped && (stages & 1)) {  // reverse state pass (one- or two-level): dh per chunk, d delta, d h0
    const int rc = run_state_pass<K, V>(B * H, bl.gc, work + bl.grp, true, stream,
                                        [&](dim3 grid, const kdn_state::GroupPlan& P) {
                                          launch_state(grid, P, dht, dh0, stream);
                                        });
    if (rc) return rc;
  }
  if (!overlapped && (stages & 2)) {
    launch_chunk(0, tasks, stream);
    KDN_CHECK_LAUNCH();
  }
  if ((stages & 12) == 12) {  // both exact stages: one launch runs each flagged chunk's solves, gradients and norm
    const int NB = B * H * NT, gx = min(NB, 256);  // one workgroup per CU fits (its LDS)
#define KDN_EXACT(ISO_)                                                                                               \
  hipLaunchKernelGGL((mem_bwd_exact_kernel<K, V, ISO_>), dim3(gx), dim3(256), 0, stream, q, k, kap, gc, dD, dW, U, W, \
                     dM, dQg, dKf, dgl, T, H, NT, NB, flags, scale, dv, dKg, dN, dq, dk, dkap, dbeta, dg, q_rstd,      \
                     k_rstd, (hm & kdn_state::HB_DD) != 0)
    if (iso) KDN_EXACT(true);
    else KDN_EXACT(false);
#undef KDN_EXACT
    KDN_CHECK_LAUNCH();
    return 0;
  }
  if (stages & 4) {  // the chunks left to the exact path: transposed solves into dv, dKg, dN
    const int NB = B * H * NT, gx = min(NB, 512);
    if (iso)
      hipLaunchKernelGGL((mem_bwd_solve_exact_kernel<K, V, true>), dim3(gx), dim3(256), 0, stream, k, kap, gc, dD, dW,
                         U, W, T, H, NT, NB, flags, dv, dKg, dN, k_rstd, (hm & kdn_state::HB_DD) != 0);
    else
      hipLaunchKernelGGL((mem_bwd_solve_exact_kernel<K, V, false>), dim3(gx), dim3(256), 0, stream, k, kap, gc, dD,
                         dW, U, W, T, H, NT, NB, flags, dv, dKg, dN, k_rstd, (hm & kdn_state::HB_DD) != 0);
    KDN_CHECK_LAUNCH();
  }
  if (stages & 8) {  // the exact path's gradients
    const int NB = B * H * NT, gx = min(NB, 512);
    if (iso)
      hipLaunchKernelGGL((mem_bwd_contrib_exact_kernel<K, V, true>), dim3(gx), dim3(256), 0, stream, q, k, kap, gc, dN,
                         dM, dQg, dKg, dKf, dgl, T, H, NT, NB, flags, scale, dq, dk, dkap, dbeta, dg, q_rstd, k_rstd);
    else
      hipLaunchKernelGGL((mem_bwd_contrib_exact_kernel<K, V, false>), dim3(gx), dim3(256), 0, stream, q, k, kap, gc,
                         dN, dM, dQg, dKg, dKf, dgl, T, H, NT, NB, flags, scale, dq, dk, dkap, dbeta, dg, q_rstd, k_rstd);
    KDN_CHECK_LAUNCH();
    if (q_rstd) {  // the in-op norm's backward for the flagged chunks' rows
      hipLaunchKernelGGL((l2norm_bwd_flagged_kernel<K>), dim3(gx), dim3(256), 0, stream, q, k, q_rstd, k_rstd, T, H,
                         NT, NB, flags, dq, dk);
      KDN_CHECK_LAUNCH();
    }
  }
  return 0;
}

}  // namespace

extern "C" {

int kdn_mem_chunk_size(void) { return C; }

int kdn_mem_state_groups(int B, int T, int H, int K, int V) {
  if (B <= 0 || T <= 0 || H <= 0) return KDN_ERR_ARG;
  if (!((K == 64 || K == 128) && (V == 64 || V == 128))) return KDN_ERR_ARG;
  return plan_groups(B * H, cdiv(T, C), K, V).NG;
}

size_t kdn_mem_saved_size(int B, int T, int H, int K, int V) {
  return (size_t)MemLayout(B, T, H, K, V).total * sizeof(float);
}

size_t kdn_mem_bwd_workspace_size(int B, int T, int H, int K, int V) {
  return (size_t)BwdLayout(B, T, H, K, V).total * sizeof(float);
}

int kdn_mem_fwd(const uint16_t* q, const uint16_t* k, const float* kappa_or_beta, int iso, const uint16_t* v,
                const float* g_cumsum, int B, int T, int H, int K, int V, float scale, const float* initial_state,
                void* saved, size_t saved_bytes, float* final_state, void* o, int o_bf16, float* q_rstd,
                float* k_rstd, int stages, hipStream_t stream) {
  if (B <= 0 || T <= 0 || H <= 0) return KDN_ERR_ARG;
  if (!((K == 64 || K == 128) && (V == 64 || V == 128))) return KDN_ERR_ARG;
  if (saved_bytes < kdn_mem_saved_size(B, T, H, K, V)) return KDN_ERR_ARG;
  if ((q_rstd == nullptr) != (k_rstd == nullptr)) return KDN_ERR_ARG;
  float* sv = (float*)saved;
#define KDN_MEM_FWD(KK, VV) \
  return mem_fwd_impl<KK, VV>(q, k, kappa_or_beta, iso, v, g_cumsum, B, T, H, scale, initial_state, sv, final_state, o, \
                              o_bf16, q_rstd, k_rstd, stages, stream)
  if (K == 128 && V == 128) KDN_MEM_FWD(128, 128);
  if (K == 64 && V == 64) KDN_MEM_FWD(64, 64);
  if (K == 128 && V == 64) KDN_MEM_FWD(128, 64);
  KDN_MEM_FWD(64, 128);
#undef KDN_MEM_FWD
}

int kdn_mem_bwd(const uint16_t* q, const uint16_t* k, const float* kappa_or_beta, int iso, const float* g_cumsum,
                int B, int T, int H, int K, int V, float scale, const void* d_o, int do_bf16,
                const float* d_final_state, const void* saved, size_t saved_bytes, void* workspace,
                size_t workspace_bytes, uint16_t* dq, uint16_t* dk, float* dkappa, float* dbeta, uint16_t* dv,
                float* dg, float* d_initial_state, const float* q_rstd, const float* k_rstd, int stages,
                hipStream_t stream) {
  if (B <= 0 || T <= 0 || H <= 0) return KDN_ERR_ARG;
  if (!((K == 64 || K == 128) && (V == 64 || V == 128))) return KDN_ERR_ARG;
  if (saved_bytes < kdn_mem_saved_size(B, T, H, K, V)) return KDN_ERR_ARG;
  if (workspace_bytes < kdn_mem_bwd_workspace_size(B, T, H, K, V)) return KDN_ERR_ARG;
  if (iso ? dbeta == nullptr : dkappa == nullptr) return KDN_ERR_ARG;
  if ((q_rstd == nullptr) != (k_rstd == nullptr)) return KDN_ERR_ARG;
  const float* sv = (const float*)saved;
  float* wk = (float*)workspace;
#define KDN_MEM_BWD(KK, VV)                                                                                          \
  do {                                                                                                               \
    if (do_bf16)                                                                                                     \
      return mem_bwd_impl<KK, VV, bf16_t>(q, k, kappa_or_beta, iso, g_cumsum, B, T, H, scale, (const bf16_t*)d_o,   \
                                          d_final_state, sv, wk, dq, dk, dkappa, dbeta, dv, dg, d_initial_state,     \
                                          q_rstd, k_rstd, stages, stream);                                           \
    return mem_bwd_impl<KK, VV, float>(q, k, kappa_or_beta, iso, g_cumsum, B, T, H, scale, (const float*)d_o,       \
                                       d_final_state, sv, wk, dq, dk, dkappa, dbeta, dv, dg, d_initial_state,        \
                                       q_rstd, k_rstd, stages, stream);                                              \
  } while (0)
  if (K == 128 && V == 128) KDN_MEM_BWD(128, 128);
  if (K == 64 && V == 64) KDN_MEM_BWD(64, 64);
  if (K == 128 && V == 64) KDN_MEM_BWD(128, 64);
  KDN_MEM_BWD(64, 128);
#undef KDN_MEM_BWD
}

}  // extern "C"
