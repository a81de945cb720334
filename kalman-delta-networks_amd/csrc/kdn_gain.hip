// Kalman gain (uncertainty) scans for iso_kdn and diag_kdn, forward and backward.
//
// The covariance recurrence p_{t-1} -> p_t is a projective (Mobius) map, so a token
// range composes into one 2x2 matrix; the reverse adjoint recurrence lambda_t ->
// lambda_{t-1} is affine.  Both are scanned in parallel and replayed per token.
//
// iso (one scalar per head; reference lit_gpt/kdn_ops/iso_kdn_chunk.py:1464-1893):
//   z = a p + w;  beta = z / (r + z);  p' = r z / (r + s z)    (s = info_scale / K)
//   One wavefront owns one (b, h) stream; lane j owns a contiguous token segment, the
//   segment maps are combined with a wave-level shuffle scan (no global carry pass).
// diag (one value per key channel; reference diag_kdn_chunk.py:373-700):
//   p_hat = alpha^2 p + w;  kappa = p_hat k / (r + sum_i p_hat_i k_i^2);
//   p' = p_hat / (1 + u p_hat),  u = s k^2 / r  (s = info_scale = K)
//   map / carry / emit passes over 64-token chunks, one workgroup per (chunk, b, h),
//   thread = key channel; the per-token cross-channel sums are wave reductions whose
//   partials are deferred to LDS so no barrier sits inside the token loop.
#include "kdn_common.h"
#include "../../include/kdn.h"

namespace {

// ----------------------------------------------------------------------------
// 2x2 map helpers (row-major m0 m1 / m2 m3).  compose(a, b) = a * b (b applied first).
// ----------------------------------------------------------------------------
struct Map2 {
  float m0, m1, m2, m3;
};
__device__ __forceinline__ Map2 map_mul(const Map2& a, const Map2& b) {
  Map2 c{a.m0 * b.m0 + a.m1 * b.m2, a.m0 * b.m1 + a.m1 * b.m3, a.m2 * b.m0 + a.m3 * b.m2,
         a.m2 * b.m1 + a.m3 * b.m3};
  const float s = fmaxf(fmaxf(fabsf(c.m0), fabsf(c.m1)), fmaxf(fabsf(c.m2), fabsf(c.m3)));
  const float inv = 1.f / fmaxf(s, 1e-30f);
  c.m0 *= inv; c.m1 *= inv; c.m2 *= inv; c.m3 *= inv;
  return c;
}
__device__ __forceinline__ float mobius(const Map2& m, float p) { return (m.m0 * p + m.m1) / (m.m2 * p + m.m3); }
__device__ __forceinline__ Map2 shfl_up_map(const Map2& m, int d) {
  return Map2{__shfl_up(m.m0, d, 64), __shfl_up(m.m1, d, 64), __shfl_up(m.m2, d, 64), __shfl_up(m.m3, d, 64)};
}

// ----------------------------------------------------------------------------
// iso gain, block per head: the block's 256-thread groups take batch rows b = g, g + GB, ...;
// thread j of a group owns tokens [j S, (j+1) S), S = ceil(T / 256).  Segment maps are
// combined by a wave shuffle scan and an LDS scan over the group's 4 waves, then replayed.
// ----------------------------------------------------------------------------
constexpr int kIsoGroup = 256;
constexpr int kIsoBatch = 16;  // tokens loaded per batch in the segment loops

__device__ __forceinline__ Map2 map_identity() { return Map2{1.f, 0.f, 0.f, 1.f}; }

// Exclusive scan of segment maps over the 256 threads of group g (later maps applied after).
__device__ __forceinline__ Map2 group_exclusive_map(Map2 M, Map2* sW, int g, int lane, int w) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const Map2 prev = shfl_up_map(M, d);
    if (lane >= d) M = map_mul(M, prev);
  }
  if (lane == 63) sW[4 * g + w] = M;
  __syncthreads();
  Map2 P = map_identity();
  for (int q = 0; q < w; ++q) P = map_mul(sW[4 * g + q], P);
  Map2 E = shfl_up_map(M, 1);
  if (lane == 0) E = map_identity();
  return map_mul(E, P);
}

// grid (H), block 256 * GB.
__global__ __launch_bounds__(1024) void iso_gain_fwd_grp_kernel(const float* __restrict__ a,
                                                                const float* __restrict__ omega,
                                                                const float* __restrict__ r,
                                                                const float* __restrict__ mu, int B, int T, int H,
                                                                float s, int unit_scale, float* __restrict__ beta,
                                                                float* __restrict__ p_prev,
                                                                float* __restrict__ final_precision) {
  __shared__ Map2 sW[16];
  const int h = blockIdx.x, GB = blockDim.x / kIsoGroup, g = threadIdx.x / kIsoGroup;
  const int j = threadIdx.x % kIsoGroup, lane = j & 63, w = j >> 6;
  const int S = (T + kIsoGroup - 1) / kIsoGroup;
  const int t0 = min(j * S, T), t1 = min(t0 + S, T);
  const float p0 = 1.f / mu[h];
  for (int b0 = 0; b0 < B; b0 += GB) {
    const int b = b0 + g;
    const bool act = b < B;
    const int64_t base = (int64_t)(act ? b : 0) * T * H + h;
    Map2 M = map_identity();
    if (act) {
      for (int tb = t0; tb < t1; tb += kIsoBatch) {
        float at[kIsoBatch], wt[kIsoBatch], rt[kIsoBatch];
#pragma unroll
        for (int u = 0; u < kIsoBatch; ++u) {
          const int64_t o = base + (int64_t)min(tb + u, t1 - 1) * H;
          at[u] = a[o], wt[u] = omega[o], rt[u] = r[o];
        }
#pragma unroll
        for (int u = 0; u < kIsoBatch; ++u)
          if (tb + u < t1) M = map_mul(Map2{rt[u] * at[u], rt[u] * wt[u], s * at[u], rt[u] + s * wt[u]}, M);
      }
    }
    const Map2 E = group_exclusive_map(M, sW, g, lane, w);
    float p = mobius(E, p0);
    if (act) {
      for (int tb = t0; tb < t1; tb += kIsoBatch) {
        float at[kIsoBatch], wt[kIsoBatch], rt[kIsoBatch];
#pragma unroll
        for (int u = 0; u < kIsoBatch; ++u) {
          const int64_t o = base + (int64_t)min(tb + u, t1 - 1) * H;
          at[u] = a[o], wt[u] = omega[o], rt[u] = r[o];
        }
#pragma unroll
        for (int u = 0; u < kIsoBatch; ++u) {
          if (tb + u >= t1) break;
          const int64_t o = base + (int64_t)(tb + u) * H;
          if (p_prev) p_prev[o] = p;
          const float z = at[u] * p + wt[u];
          const float gg = z / (rt[u] + z);
          beta[o] = gg;
          p = unit_scale ? rt[u] * gg : rt[u] * z / (rt[u] + s * z);
        }
      }
      if (final_precision && t0 < T && t1 == T) final_precision[(int64_t)b * H + h] = 1.f / p;
    }
    __syncthreads();  // sW is reused by the next batch rows
  }
}

// grid (H), block 256 * GB.  lambda_{t-1} = A_t lambda_t + B_t (reverse), lambda_T = 0.
__global__ __launch_bounds__(1024) void iso_gain_bwd_grp_kernel(
    const float* __restrict__ a, const float* __restrict__ omega, const float* __restrict__ r,
    const float* __restrict__ mu, const float* __restrict__ dbeta, const float* __restrict__ p_prev, int B, int T,
    int H, float s, int unit_scale, float* __restrict__ da, float* __restrict__ domega, float* __restrict__ dr,
    float* __restrict__ dmu) {
  __shared__ float sA[16], sB[16], sMu[4];
  const int h = blockIdx.x, GB = blockDim.x / kIsoGroup, g = threadIdx.x / kIsoGroup;
  const int j = threadIdx.x % kIsoGroup, lane = j & 63, w = j >> 6;
  const int S = (T + kIsoGroup - 1) / kIsoGroup;
  const int t0 = min(j * S, T), t1 = min(t0 + S, T);
  const float muh = mu[h];
  float dmu_acc = 0.f;
  for (int b0 = 0; b0 < B; b0 += GB) {
    const int b = b0 + g;
    const bool act = b < B;
    const int64_t base = (int64_t)(act ? b : 0) * T * H + h;
    float Aseg = 1.f, Bseg = 0.f;
    if (act) {
      for (int te = t1; te > t0; te -= kIsoBatch) {  // tokens te-1 down to te-kIsoBatch
        float at[kIsoBatch], wt[kIsoBatch], rt[kIsoBatch], dl[kIsoBatch], pp[kIsoBatch];
#pragma unroll
        for (int u = 0; u < kIsoBatch; ++u) {
          const int64_t o = base + (int64_t)max(te - 1 - u, t0) * H;
          at[u] = a[o], wt[u] = omega[o], rt[u] = r[o], dl[u] = dbeta[o], pp[u] = p_prev[o];
        }
#pragma unroll
        for (int u = 0; u < kIsoBatch; ++u) {
          if (te - 1 - u < t0) break;
          const float z = at[u] * pp[u] + wt[u];
          const float ig = 1.f / (rt[u] + z), ip = 1.f / (rt[u] + s * z);
          const float At = at[u] * rt[u] * rt[u] * ip * ip;
          const float Bt = at[u] * dl[u] * rt[u] * ig * ig;
          Bseg = At * Bseg + Bt;
          Aseg = At * Aseg;
        }
      }
    }
    // exclusive suffix scan over the group: lambda after this thread's segment
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const float An = __shfl_down(Aseg, d, 64), Bn = __shfl_down(Bseg, d, 64);
      if (lane + d < 64) {
        Bseg = Aseg * Bn + Bseg;
        Aseg = Aseg * An;
      }
    }
    if (lane == 0) {
      sA[4 * g + w] = Aseg;
      sB[4 * g + w] = Bseg;
    }
    __syncthreads();
    float lam = 0.f;  // lambda entering the later waves' segments, applied from the last wave back
    for (int q = 3; q > w; --q) lam = sA[4 * g + q] * lam + sB[4 * g + q];
    {
      const float An = __shfl_down(Aseg, 1, 64), Bn = __shfl_down(Bseg, 1, 64);
      if (lane < 63) lam = An * lam + Bn;
    }
    if (act) {
      for (int te = t1; te > t0; te -= kIsoBatch) {
        float at[kIsoBatch], wt[kIsoBatch], rt[kIsoBatch], dl[kIsoBatch], pp[kIsoBatch];
#pragma unroll
        for (int u = 0; u < kIsoBatch; ++u) {
          const int64_t o = base + (int64_t)max(te - 1 - u, t0) * H;
          at[u] = a[o], wt[u] = omega[o], rt[u] = r[o], dl[u] = dbeta[o], pp[u] = p_prev[o];
        }
#pragma unroll
        for (int u = 0; u < kIsoBatch; ++u) {
          if (te - 1 - u < t0) break;
          const int64_t o = base + (int64_t)(te - 1 - u) * H;
          const float z = at[u] * pp[u] + wt[u];
          const float ig = 1.f / (rt[u] + z);
          const float ig2 = ig * ig;
          float zbar, drt;
          if (unit_scale) {
            zbar = (dl[u] + rt[u] * lam) * rt[u] * ig2;
            drt = z * (lam * z - dl[u]) * ig2;
          } else {
            const float ip = 1.f / (rt[u] + s * z);
            const float ip2 = ip * ip;
            zbar = dl[u] * rt[u] * ig2 + lam * rt[u] * rt[u] * ip2;
            drt = -dl[u] * z * ig2 + lam * s * z * z * ip2;
          }
          da[o] = zbar * pp[u];
          domega[o] = zbar;
          dr[o] = drt;
          lam = at[u] * zbar;
        }
      }
      if (j == 0) dmu_acc += -lam / (muh * muh);
    }
    __syncthreads();  // sA / sB are reused by the next batch rows
  }
  if (j == 0) sMu[g] = dmu_acc;
  __syncthreads();
  if (threadIdx.x == 0 && dmu) {
    float tot = 0.f;
    for (int q = 0; q < GB; ++q) tot += sMu[q];
    dmu[h] = tot;
  }
}

// ----------------------------------------------------------------------------
// diag gain.  Layouts: k, alpha, omega, kappa, p_prev [B,T,H,K]; r, D [B,T,H].
// maps [B,H,NT,K,4], carry [B,H,NT,K]; block = K rounded up to 64, thread = channel.
// ----------------------------------------------------------------------------
constexpr int kGainChunk = 64;

__global__ __launch_bounds__(256) void diag_gain_map_kernel(const float* __restrict__ k, const float* __restrict__ alpha,
                                                            const float* __restrict__ omega, const float* __restrict__ r,
                                                            int T, int H, int K, int NT, float s,
                                                            float* __restrict__ maps) {
  const int nt = blockIdx.x, bh = blockIdx.y, b = bh / H, h = bh % H, i = threadIdx.x;
  if (i >= K) return;
  const int t0 = nt * kGainChunk, t1 = min(t0 + kGainChunk, T);
  Map2 M{1.f, 0.f, 0.f, 1.f};
  for (int t = t0; t < t1; ++t) {
    const int64_t o = (((int64_t)b * T + t) * H + h) * K + i;
    const float kt = k[o], al = alpha[o], wt = omega[o];
    const float rt = r[((int64_t)b * T + t) * H + h];
    const float a2 = al * al, u = s * kt * kt / rt;
    M = map_mul(Map2{a2, wt, u * a2, 1.f + u * wt}, M);
  }
  float* dst = maps + ((((int64_t)b * H + h) * NT + nt) * K + i) * 4;
  dst[0] = M.m0; dst[1] = M.m1; dst[2] = M.m2; dst[3] = M.m3;
}

// p0 from initial precision: prec_mode 0 -> [H], 1 -> [B,H,K]
__global__ __launch_bounds__(256) void diag_gain_carry_kernel(const float* __restrict__ maps, const float* __restrict__ prec0,
                                                              int prec_mode, int H, int K, int NT,
                                                              float* __restrict__ carry, float* __restrict__ final_prec) {
  const int bh = blockIdx.x, b = bh / H, h = bh % H, i = threadIdx.x;
  if (i >= K) return;
  float p = 1.f / (prec_mode == 0 ? prec0[h] : prec0[((int64_t)b * H + h) * K + i]);
  const int64_t cb = ((int64_t)b * H + h) * NT;
  for (int nt = 0; nt < NT; ++nt) {
    carry[(cb + nt) * K + i] = p;
    const float* m = maps + ((cb + nt) * K + i) * 4;
    p = (m[0] * p + m[1]) / (m[2] * p + m[3]);
  }
  if (final_prec) final_prec[((int64_t)b * H + h) * K + i] = 1.f / p;
}

__global__ __launch_bounds__(256) void diag_gain_emit_kernel(const float* __restrict__ k, const float* __restrict__ alpha,
                                                             const float* __restrict__ omega, const float* __restrict__ r,
                                                             const float* __restrict__ carry, int T, int H, int K,
                                                             int NT, float s, float* __restrict__ kappa,
                                                             float* __restrict__ p_prev, float* __restrict__ Dsave) {
  __shared__ float num[kGainChunk][257];
  __shared__ float part[kGainChunk][4];
  const int nt = blockIdx.x, bh = blockIdx.y, b = bh / H, h = bh % H, i = threadIdx.x;
  const int lane = i & 63, w = i >> 6;
  const int t0 = nt * kGainChunk, L = min(kGainChunk, T - t0);
  const bool act = i < K;
  float p = act ? carry[(((int64_t)b * H + h) * NT + nt) * K + i] : 0.f;
  for (int t = 0; t < L; ++t) {
    const int64_t o = (((int64_t)b * T + t0 + t) * H + h) * K + i;
    const float rt = r[((int64_t)b * T + t0 + t) * H + h];
    float kt = 0.f, ph = 0.f;
    if (act) {
      kt = k[o];
      const float al = alpha[o];
      ph = al * al * p + omega[o];
      if (p_prev) p_prev[o] = p;
      num[t][i] = ph * kt;
      p = ph / (1.f + s * kt * kt / rt * ph);
    }
    const float ps = wave_sum(ph * kt * kt);
    if (lane == 0) part[t][w] = ps;
  }
  __syncthreads();
  const int nw = (blockDim.x + 63) >> 6;
  if (act) {
    for (int t = 0; t < L; ++t) {
      float D = r[((int64_t)b * T + t0 + t) * H + h];
      for (int j = 0; j < nw; ++j) D += part[t][j];
      kappa[(((int64_t)b * T + t0 + t) * H + h) * K + i] = num[t][i] / D;
    }
  }
  if (Dsave && i < L) {
    float D = r[((int64_t)b * T + t0 + i) * H + h];
    for (int j = 0; j < nw; ++j) D += part[i][j];
    Dsave[((int64_t)b * T + t0 + i) * H + h] = D;
  }
}

// Backward map pass: affine (A, B) per channel over the chunk, plus G_t = sum_i dkappa_i kappa_i.
__global__ __launch_bounds__(256) void diag_gain_bwd_map_kernel(
    const float* __restrict__ k, const float* __restrict__ alpha, const float* __restrict__ omega,
    const float* __restrict__ r, const float* __restrict__ dkappa, const float* __restrict__ p_prev,
    const float* __restrict__ Dsave, int T, int H, int K, int NT, float s, float* __restrict__ ab,
    float* __restrict__ Gsave) {
  __shared__ float part[kGainChunk][4];
  const int nt = blockIdx.x, bh = blockIdx.y, b = bh / H, h = bh % H, i = threadIdx.x;
  const int lane = i & 63, w = i >> 6, nw = (blockDim.x + 63) >> 6;
  const int t0 = nt * kGainChunk, L = min(kGainChunk, T - t0);
  const bool act = i < K;
  for (int t = 0; t < L; ++t) {
    float g = 0.f;
    if (act) {
      const int64_t o = (((int64_t)b * T + t0 + t) * H + h) * K + i;
      const float al = alpha[o];
      const float ph = al * al * p_prev[o] + omega[o];
      g = dkappa[o] * ph * k[o] / Dsave[((int64_t)b * T + t0 + t) * H + h];
    }
    g = wave_sum(g);
    if (lane == 0) part[t][w] = g;
  }
  __syncthreads();
  float Aacc = 1.f, Bacc = 0.f;
  if (act) {
    for (int t = L - 1; t >= 0; --t) {
      const int64_t o = (((int64_t)b * T + t0 + t) * H + h) * K + i;
      const int64_t ot = ((int64_t)b * T + t0 + t) * H + h;
      float G = 0.f;
      for (int j = 0; j < nw; ++j) G += part[t][j];
      const float kt = k[o], al = alpha[o], a2 = al * al;
      const float ph = a2 * p_prev[o] + omega[o];
      const float D = Dsave[ot], rt = r[ot];
      const float hh = 1.f + s * kt * kt / rt * ph;
      const float pbar = dkappa[o] * kt / D - kt * kt * G / D;
      const float At = a2 / (hh * hh);
      Bacc = At * Bacc + a2 * pbar;
      Aacc = At * Aacc;
    }
    float* dst = ab + ((((int64_t)b * H + h) * NT + nt) * K + i) * 2;
    dst[0] = Aacc;
    dst[1] = Bacc;
  }
  if (Gsave && i < L) {
    float G = 0.f;
    for (int j = 0; j < nw; ++j) G += part[i][j];
    Gsave[((int64_t)b * T + t0 + i) * H + h] = G;
  }
}

// lambda carry (reverse over chunks). lam_end from d_final_precision: dL/dp_T = -dprec / p_T^2.
__global__ __launch_bounds__(256) void diag_gain_bwd_carry_kernel(const float* __restrict__ ab,
                                                                  const float* __restrict__ d_final_prec,
                                                                  const float* __restrict__ final_prec, int H, int K,
                                                                  int NT, float* __restrict__ carry) {
  const int bh = blockIdx.x, i = threadIdx.x;
  if (i >= K) return;
  float lam = 0.f;
  if (d_final_prec) {
    const float c = final_prec[(int64_t)bh * K + i];
    lam = -d_final_prec[(int64_t)bh * K + i] * c * c;  // p = 1/c -> dL/dp = -c^2 dL/dc
  }
  const int64_t cb = (int64_t)bh * NT;
  for (int nt = NT - 1; nt >= 0; --nt) {
    carry[(cb + nt) * K + i] = lam;
    const float* m = ab + ((cb + nt) * K + i) * 2;
    lam = m[0] * lam + m[1];
  }
}

__global__ __launch_bounds__(256) void diag_gain_bwd_emit_kernel(
    const float* __restrict__ k, const float* __restrict__ alpha, const float* __restrict__ omega,
    const float* __restrict__ r, const float* __restrict__ dkappa, const float* __restrict__ p_prev,
    const float* __restrict__ Dsave, const float* __restrict__ Gsave, const float* __restrict__ carry,
    const bf16_t* __restrict__ omega_raw, const bf16_t* __restrict__ r_raw, const float* __restrict__ prec0,
    int prec_mode, int T, int H, int K, int NT, float s, float* __restrict__ dk, float* __restrict__ dalpha,
    bf16_t* __restrict__ domega_raw, bf16_t* __restrict__ dr_raw, float* __restrict__ dprec_part) {
  __shared__ float part[kGainChunk][4];
  __shared__ float red[16];
  const int nt = blockIdx.x, bh = blockIdx.y, b = bh / H, h = bh % H, i = threadIdx.x;
  const int lane = i & 63, w = i >> 6, nw = (blockDim.x + 63) >> 6;
  const int t0 = nt * kGainChunk, L = min(kGainChunk, T - t0);
  const bool act = i < K;
  float lam = act ? carry[(((int64_t)b * H + h) * NT + nt) * K + i] : 0.f;
  for (int t = L - 1; t >= 0; --t) {
    const int64_t ot = ((int64_t)b * T + t0 + t) * H + h;
    float urr = 0.f;
    if (act) {
      const int64_t o = ot * K + i;
      const float kt = k[o], al = alpha[o], a2 = al * al, pp = p_prev[o], dki = dkappa[o];
      const float ph = a2 * pp + omega[o];
      const float D = Dsave[ot], G = Gsave[ot], rt = r[ot];
      const float u = s * kt * kt / rt;
      const float hh = 1.f + u * ph;
      const float pnext = ph / hh;
      const float pbar_gain = dki * kt / D - kt * kt * G / D;
      const float pbar = pbar_gain + lam / (hh * hh);
      const float ubar = -lam * pnext * pnext;
      dk[o] = dki * ph / D - 2.f * ph * kt * G / D + ubar * (2.f * s * kt / rt);
      dalpha[o] = 2.f * al * pp * pbar;
      domega_raw[o] = f2bf(pbar * sigmoidf(bf2f(omega_raw[o])));
      urr = ubar * (-s * kt * kt / (rt * rt));
      lam = a2 * pbar;
    }
    urr = wave_sum(urr);
    if (lane == 0) part[t][w] = urr;
  }
  __syncthreads();
  if (i < L) {
    const int64_t ot = ((int64_t)b * T + t0 + i) * H + h;
    float drt = -Gsave[ot] / Dsave[ot];
    for (int j = 0; j < nw; ++j) drt += part[i][j];
    dr_raw[ot] = f2bf(drt * sigmoidf(bf2f(r_raw[ot])));
  }
  if (nt == 0 && dprec_part) {
    // lam now holds dL/dp_{-1}; p_{-1} = 1/c  ->  dL/dc = -lam p^2
    float contrib = 0.f;
    if (act) {
      const float c = prec_mode == 0 ? prec0[h] : prec0[((int64_t)b * H + h) * K + i];
      const float p0 = 1.f / c;
      contrib = -lam * p0 * p0;
      if (prec_mode == 1) dprec_part[((int64_t)b * H + h) * K + i] = contrib;
    }
    if (prec_mode == 0) {
      const float tot = block_sum(contrib, red);
      if (i == 0) dprec_part[(int64_t)b * H + h] = tot;
    }
  }
}

// dprec[h] = sum_b part[b, h]
__global__ void sum_over_batch_kernel(const float* __restrict__ part, int B, int H, float* __restrict__ out) {
  const int h = blockIdx.x * blockDim.x + threadIdx.x;
  if (h >= H) return;
  float s = 0.f;
  for (int b = 0; b < B; ++b) s += part[(int64_t)b * H + h];
  out[h] = s;
}

inline int cdiv(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }
inline int gain_block(int K) { return ((K + 63) / 64) * 64; }

}  // namespace

extern "C" {

int kdn_iso_gain_fwd(const float* a, const float* omega, const float* r, const float* initial_precision, int B, int T,
                     int H, float posterior_scale, float* beta, float* p_prev, float* final_precision,
                     hipStream_t stream) {
  if (B < 0 || T < 0 || H <= 0 || !(posterior_scale > 0.f)) return KDN_ERR_ARG;
  if (B == 0 || T == 0) return 0;
  const int GB = B < 4 ? B : 4;
  hipLaunchKernelGGL(iso_gain_fwd_grp_kernel, dim3(H), dim3(kIsoGroup * GB), 0, stream, a, omega, r,
                     initial_precision, B, T, H, posterior_scale, posterior_scale == 1.f ? 1 : 0, beta, p_prev,
                     final_precision);
  KDN_CHECK_LAUNCH();
  return 0;
}

int kdn_iso_gain_bwd(const float* a, const float* omega, const float* r, const float* initial_precision,
                     const float* dbeta, const float* p_prev, int B, int T, int H, float posterior_scale, float* da,
                     float* domega, float* dr, float* d_initial_precision, hipStream_t stream) {
  if (B < 0 || T < 0 || H <= 0 || !(posterior_scale > 0.f)) return KDN_ERR_ARG;
  if (B == 0 || T == 0) return 0;
  const int GB = B < 4 ? B : 4;
  hipLaunchKernelGGL(iso_gain_bwd_grp_kernel, dim3(H), dim3(kIsoGroup * GB), 0, stream, a, omega, r,
                     initial_precision, dbeta, p_prev, B, T, H, posterior_scale, posterior_scale == 1.f ? 1 : 0, da,
                     domega, dr, d_initial_precision);
  KDN_CHECK_LAUNCH();
  return 0;
}

size_t kdn_diag_gain_workspace_size(int B, int T, int H, int K) {
  const int64_t NT = cdiv(T, kGainChunk);
  // maps (4) + carry (1) per (b, h, chunk, channel), plus [B,H,K] precision partials
  return (size_t)((int64_t)B * H * NT * K * 5 + (int64_t)B * H * K) * sizeof(float);
}

int kdn_diag_gain_fwd(const float* k, const float* alpha, const float* omega, const float* r,
                      const float* initial_precision, int prec_mode, int B, int T, int H, int K, float info_scale,
                      float* kappa, float* p_prev, float* D, float* final_precision, void* workspace,
                      size_t workspace_bytes, hipStream_t stream) {
  if (B <= 0 || T <= 0 || H <= 0 || K <= 0 || K > 256 || (prec_mode != 0 && prec_mode != 1)) return KDN_ERR_ARG;
  if (workspace_bytes < kdn_diag_gain_workspace_size(B, T, H, K)) return KDN_ERR_ARG;
  const int NT = cdiv(T, kGainChunk);
  float* maps = (float*)workspace;
  float* carry = maps + (int64_t)B * H * NT * K * 4;
  const int bs = gain_block(K);
  hipLaunchKernelGGL(diag_gain_map_kernel, dim3(NT, B * H), dim3(bs), 0, stream, k, alpha, omega, r, T, H, K, NT,
                     info_scale, maps);
  hipLaunchKernelGGL(diag_gain_carry_kernel, dim3(B * H), dim3(bs), 0, stream, maps, initial_precision, prec_mode, H, K,
                     NT, carry, final_precision);
  hipLaunchKernelGGL(diag_gain_emit_kernel, dim3(NT, B * H), dim3(bs), 0, stream, k, alpha, omega, r, carry, T, H, K,
                     NT, info_scale, kappa, p_prev, D);
  KDN_CHECK_LAUNCH();
  return 0;
}

int kdn_diag_gain_bwd(const float* k, const float* alpha, const float* omega, const float* r,
                      const float* initial_precision, int prec_mode, const float* dkappa, const float* p_prev,
                      const float* D, const float* final_precision, const float* d_final_precision,
                      const uint16_t* omega_raw, const uint16_t* r_raw, int B, int T, int H, int K, float info_scale,
                      float* dk, float* dalpha, uint16_t* domega_raw, uint16_t* dr_raw, float* d_initial_precision,
                      float* G_scratch, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (B <= 0 || T <= 0 || H <= 0 || K <= 0 || K > 256 || (prec_mode != 0 && prec_mode != 1)) return KDN_ERR_ARG;
  if (workspace_bytes < kdn_diag_gain_workspace_size(B, T, H, K)) return KDN_ERR_ARG;
  if (d_final_precision && !final_precision) return KDN_ERR_ARG;
  const int NT = cdiv(T, kGainChunk);
  float* ab = (float*)workspace;                     // [B,H,NT,K,2]
  float* carry = ab + (int64_t)B * H * NT * K * 4;   // [B,H,NT,K]
  float* dpart = carry + (int64_t)B * H * NT * K;    // [B,H] or [B,H,K]
  const int bs = gain_block(K);
  hipLaunchKernelGGL(diag_gain_bwd_map_kernel, dim3(NT, B * H), dim3(bs), 0, stream, k, alpha, omega, r, dkappa, p_prev,
                     D, T, H, K, NT, info_scale, ab, G_scratch);
  hipLaunchKernelGGL(diag_gain_bwd_carry_kernel, dim3(B * H), dim3(bs), 0, stream, ab, d_final_precision,
                     final_precision, H, K, NT, carry);
  float* dpart_out = d_initial_precision ? (prec_mode == 1 ? d_initial_precision : dpart) : nullptr;
  hipLaunchKernelGGL(diag_gain_bwd_emit_kernel, dim3(NT, B * H), dim3(bs), 0, stream, k, alpha, omega, r, dkappa,
                     p_prev, D, G_scratch, carry, omega_raw, r_raw, initial_precision, prec_mode, T, H, K, NT,
                     info_scale, dk, dalpha, domega_raw, dr_raw, dpart_out);
  if (d_initial_precision && prec_mode == 0)
    hipLaunchKernelGGL(sum_over_batch_kernel, dim3(cdiv(H, 256)), dim3(256), 0, stream, dpart, B, H,
                       d_initial_precision);
  KDN_CHECK_LAUNCH();
  return 0;
}

}  // extern "C"
