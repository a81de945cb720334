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
#include <algorithm>
#include <mutex>

#include "kdn_common.h"
#include "kdn_iso_gain.h"
#include "../../include/kdn.h"

namespace {

// ----------------------------------------------------------------------------
// iso gain, standalone entry points: map / emit forward, map / carry / emit backward over 64-token
// chunks (the emit forward and the backward map are shared with the fused front, kdn_iso_gain.h).
// Workspace (5 floats per (b, h, chunk)): forward maps [B*H][NC] x 4 floats; backward maps [B*H][NC] x 2
// floats, then lambda after each chunk [B*H][NC].
// ----------------------------------------------------------------------------

// grid (NC, B), block 256, dynamic LDS 3 * 64 * H floats + 4 * H maps.
__global__ __launch_bounds__(256) void iso_gain_map_kernel(const float* __restrict__ a, const float* __restrict__ omega,
                                                           const float* __restrict__ r, int T, int H, int NC, float s,
                                                           float4* __restrict__ maps) {
  extern __shared__ float sm[];
  float *sa = sm, *sw = sm + kIsoChunk * H, *sr = sm + 2 * kIsoChunk * H;
  Map2* sub = reinterpret_cast<Map2*>(sm + 3 * kIsoChunk * H);
  const int n = blockIdx.x, b = blockIdx.y, t0 = n * kIsoChunk, L = min(kIsoChunk, T - t0);
  stage_bth_n<3>({a, omega, r}, b, T, H, t0, L, sa);
  __syncthreads();
  constexpr int SL = kIsoChunk / kIsoSub;
  for (int hq = threadIdx.x; hq < kIsoSub * H; hq += blockDim.x) {
    const int h = hq / kIsoSub, q = hq % kIsoSub;
    Map2 M = map_identity();
    for (int t = q * SL; t < min(L, (q + 1) * SL); ++t)
      M = map_mul_r(token_map(sa[t * H + h], sw[t * H + h], sr[t * H + h], s), M);
    sub[hq] = M;
  }
  __syncthreads();
  for (int h = threadIdx.x; h < H; h += blockDim.x) {
    Map2 M = sub[kIsoSub * h];
    for (int q = 1; q < kIsoSub; ++q) M = map_mul_r(sub[kIsoSub * h + q], M);
    maps[((int64_t)b * H + h) * NC + n] = float4{M.m0, M.m1, M.m2, M.m3};
  }
}

// grid (H), block 64 * GB (GB = min(B, 16)): wave g scans batch rows b = g, g + GB, ... from the
// last chunk back; lambda after each chunk goes to `carry`.  lambda after the last token is the
// cotangent of p_T: with final precision c_T = 1/p_T and its cotangent dc, lambda_T = -dc c_T^2
// (zero without dc).  d mu = -lambda_0 / mu^2, summed over b for a per-head mu (prec_mode 0), per
// batch row for mu [B,H] (prec_mode 1).
__global__ __launch_bounds__(1024) void iso_gain_bwd_carry_kernel(const float2* __restrict__ maps,
                                                                  const float* __restrict__ mu, int prec_mode, int B,
                                                                  int H, int NC, const float* __restrict__ fprec,
                                                                  const float* __restrict__ dfprec,
                                                                  float* __restrict__ carry, float* __restrict__ dmu) {
  __shared__ float sMu[16];
  const int h = blockIdx.x, lane = threadIdx.x & 63, g = threadIdx.x >> 6, GB = blockDim.x >> 6;
  float dmu_acc = 0.f;
  for (int b = g; b < B; b += GB) {
    const int64_t bh = (int64_t)b * H + h;
    float lam = dfprec ? -dfprec[bh] * fprec[bh] * fprec[bh] : 0.f;  // lambda after the last token
    for (int c1 = NC; c1 > 0; c1 -= 64) {
      const int c = c1 - 1 - lane;  // lane 0 = latest chunk of this group
      float2 F{1.f, 0.f};
      if (c >= 0) F = maps[bh * NC + c];
      // inclusive scan over lanes: lane j composes chunks c1-1 ... c1-1-j (latest applied first)
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const float Ap = __shfl_up(F.x, d, 64), Bp = __shfl_up(F.y, d, 64);
        if (lane >= d) F = aff_compose(F, float2{Ap, Bp});
      }
      float Ae = __shfl_up(F.x, 1, 64), Be = __shfl_up(F.y, 1, 64);
      if (lane == 0) Ae = 1.f, Be = 0.f;
      if (c >= 0) carry[bh * NC + c] = Ae * lam + Be;  // lambda after chunk c
      lam = __shfl(F.x, 63, 64) * lam + __shfl(F.y, 63, 64);
    }
    if (prec_mode) {
      if (lane == 0 && dmu) dmu[bh] = -lam / (mu[bh] * mu[bh]);
    } else if (lane == 0) {
      dmu_acc += -lam / (mu[h] * mu[h]);
    }
  }
  if (prec_mode) return;
  if (lane == 0) sMu[g] = dmu_acc;
  __syncthreads();
  if (threadIdx.x == 0 && dmu) {
    float tot = 0.f;
    for (int q = 0; q < GB; ++q) tot += sMu[q];
    dmu[h] = tot;
  }
}

// grid (NC, B), block 256, dynamic LDS 8 * 64 * H floats + 2 * 4 * H.
__global__ __launch_bounds__(256) void iso_gain_bwd_emit_kernel(
    const float* __restrict__ a, const float* __restrict__ omega, const float* __restrict__ r,
    const float* __restrict__ dbeta, const float* __restrict__ p_prev, int T, int H, int NC, float s, int unit_scale,
    const float* __restrict__ carry, float* __restrict__ da, float* __restrict__ domega, float* __restrict__ dr) {
  extern __shared__ float sm[];
  float *sa = sm, *sw = sm + kIsoChunk * H, *sr = sm + 2 * kIsoChunk * H, *sd = sm + 3 * kIsoChunk * H,
        *sp = sm + 4 * kIsoChunk * H, *oa = sm + 5 * kIsoChunk * H, *ow = sm + 6 * kIsoChunk * H,
        *orr = sm + 7 * kIsoChunk * H;
  float2* sub = reinterpret_cast<float2*>(sm + 8 * kIsoChunk * H);
  const int n = blockIdx.x, b = blockIdx.y, t0 = n * kIsoChunk, L = min(kIsoChunk, T - t0);
  stage_bth_n<5>({a, omega, r, dbeta, p_prev}, b, T, H, t0, L, sa);
  __syncthreads();
  constexpr int SL = kIsoChunk / kIsoSub;
  for (int hq = threadIdx.x; hq < kIsoSub * H; hq += blockDim.x) {
    const int h = hq / kIsoSub, q = hq % kIsoSub;
    float2 F{1.f, 0.f};
    for (int t = min(L, (q + 1) * SL) - 1; t >= q * SL; --t) {
      const int e = t * H + h;
      F = aff_compose(token_aff(sa[e], sw[e], sr[e], sd[e], sp[e], s), F);  // earlier token applied after
    }
    sub[hq] = F;
  }
  __syncthreads();
  for (int hq = threadIdx.x; hq < kIsoSub * H; hq += blockDim.x) {
    const int h = hq / kIsoSub, q = hq % kIsoSub;
    float lam = carry[((int64_t)b * H + h) * NC + n];  // lambda after the chunk
    for (int q2 = kIsoSub - 1; q2 > q; --q2) {
      const float2 F = sub[kIsoSub * h + q2];
      lam = F.x * lam + F.y;
    }
    for (int t = min(L, (q + 1) * SL) - 1; t >= q * SL; --t) {
      const int e = t * H + h;
      lam = token_grad(sa[e], sw[e], sr[e], sd[e], sp[e], lam, s, unit_scale != 0, oa[e], ow[e], orr[e]);
    }
  }
  __syncthreads();
  store_bth(da, b, T, H, t0, L, oa);
  store_bth(domega, b, T, H, t0, L, ow);
  store_bth(dr, b, T, H, t0, L, orr);
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

// ----------------------------------------------------------------------------
// Vectorised diag gain (K % 4 == 0, K/4 | 64): a thread owns CPT = 4 consecutive channels of one
// (b, h, chunk) tile; TPT = K/CPT threads per tile, tiles ordered with h fastest.  Loads and
// stores are 16-byte vectors; the per-token cross-channel sums are shuffles over the tile's
// TPT lanes.  Same workspace layouts as the per-channel kernels above.  Four channels per thread
// (rather than eight) double the waves in flight: these passes wait on loads, not arithmetic.
// ----------------------------------------------------------------------------
constexpr int kCPT = 4;  // channels per thread
__device__ __forceinline__ void ldcf(const float* p, float* f) {
#pragma unroll
  for (int q = 0; q < kCPT / 4; ++q) {
    const float4 a = reinterpret_cast<const float4*>(p)[q];
    f[4 * q] = a.x, f[4 * q + 1] = a.y, f[4 * q + 2] = a.z, f[4 * q + 3] = a.w;
  }
}
__device__ __forceinline__ void stcf(float* p, const float* f) {
#pragma unroll
  for (int q = 0; q < kCPT / 4; ++q) reinterpret_cast<float4*>(p)[q] = float4{f[4 * q], f[4 * q + 1], f[4 * q + 2], f[4 * q + 3]};
}
// kCPT bf16 values <-> floats
__device__ __forceinline__ void ldc_bf16(const bf16_t* p, float* f) {
  const uint2 v = *reinterpret_cast<const uint2*>(p);
  f[0] = __uint_as_float(v.x << 16), f[1] = __uint_as_float(v.x & 0xffff0000u);
  f[2] = __uint_as_float(v.y << 16), f[3] = __uint_as_float(v.y & 0xffff0000u);
}
__device__ __forceinline__ void stc_bf16(bf16_t* p, const float* f) {
  *reinterpret_cast<uint2*>(p) = uint2{(uint32_t)f2bf(f[0]) | ((uint32_t)f2bf(f[1]) << 16),
                                       (uint32_t)f2bf(f[2]) | ((uint32_t)f2bf(f[3]) << 16)};
}
// Sum over the tpt (a power of two <= 64) consecutive lanes of a tile, all of them active, every lane
// getting the total.  The same additions as the xor butterfly x += x[lane ^ o], o = 1, 2, 4, ...: after
// the quad steps all lanes of a quad hold the same value, so the mirrors add the same partner sums as
// lane ^ 4 and lane ^ 8 would, and the result is bit-identical to the butterfly's.
__device__ __forceinline__ float tile_sum(float x, int tpt) {
  if (tpt >= 2) x = dpp_add<kDppXor1>(x);
  if (tpt >= 4) x = dpp_add<kDppXor2>(x);
  if (tpt >= 8) x = dpp_add<kDppHalfMirror>(x);
  if (tpt >= 16) x = dpp_add<kDppMirror>(x);
  if (tpt >= 32) x = swz16_add(x);
  if (tpt >= 64) x += __shfl_xor(x, 32, 64);
  return x;
}
// Vectorised path: one tile = (b, h, 16-token chunk) x K channels, K/kCPT threads per tile, kCPT
// channels per thread.  Short chunks give B*H*T/16 * K/8 threads (enough waves to cover load latency on
// every CU); each thread issues the loads of NB tokens before it computes on them.
constexpr int kVecChunk = 16;
struct GainTile {
  int b, h, nt, i0, sub, t0, t1;
  bool ok;
};
__device__ __forceinline__ GainTile gain_tile(int B, int T, int H, int K, int NT) {
  const int tpt = K / kCPT, tpb = 256 / tpt;
  const int64_t gt = (int64_t)blockIdx.x * tpb + threadIdx.x / tpt;
  GainTile g;
  g.ok = gt < (int64_t)B * NT * H;
  const int64_t gg = g.ok ? gt : 0;
  g.h = (int)(gg % H);
  const int64_t bn = gg / H;
  g.nt = (int)(bn % NT);
  g.b = (int)(bn / NT);
  g.sub = threadIdx.x % tpt;
  g.i0 = kCPT * g.sub;
  g.t0 = g.nt * kVecChunk;
  g.t1 = min(g.t0 + kVecChunk, T);
  return g;
}
__device__ __forceinline__ int64_t gain_row(const GainTile& g, int T, int H, int t) {
  return ((int64_t)g.b * T + t) * H + g.h;
}

__global__ __launch_bounds__(256) void diag_gain_map_v_kernel(const float* __restrict__ k, const float* __restrict__ alpha,
                                                              const float* __restrict__ omega, const float* __restrict__ r,
                                                              int B, int T, int H, int K, int NT, float s,
                                                              float* __restrict__ maps) {
  constexpr int NB = 4;
  const GainTile g = gain_tile(B, T, H, K, NT);
  if (!g.ok) return;
  Map2 M[kCPT];
#pragma unroll
  for (int j = 0; j < kCPT; ++j) M[j] = Map2{1.f, 0.f, 0.f, 1.f};
  for (int t = g.t0; t < g.t1; t += NB) {
    float kt[NB][kCPT], al[NB][kCPT], wt[NB][kCPT], ir[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int64_t row = gain_row(g, T, H, min(t + u, g.t1 - 1));
      ldcf(k + row * K + g.i0, kt[u]);
      ldcf(alpha + row * K + g.i0, al[u]);
      ldcf(omega + row * K + g.i0, wt[u]);
      ir[u] = r[row];
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      if (t + u >= g.t1) break;
      const float iru = 1.f / ir[u];
#pragma unroll
      for (int j = 0; j < kCPT; ++j) {
        const float a2 = al[u][j] * al[u][j], uu = s * kt[u][j] * kt[u][j] * iru;
        M[j] = map_mul(Map2{a2, wt[u][j], uu * a2, 1.f + uu * wt[u][j]}, M[j]);
      }
    }
  }
  float4* dst = reinterpret_cast<float4*>(maps + ((((int64_t)g.b * H + g.h) * NT + g.nt) * K + g.i0) * 4);
#pragma unroll
  for (int j = 0; j < kCPT; ++j) dst[j] = float4{M[j].m0, M[j].m1, M[j].m2, M[j].m3};
}

// The prior precision c of channel i of stream (b, h): prec_mode 0 -> prec0[h] ([H] values), 1 -> [B,H,K]
// values, 2 -> prec0 holds the frontend's mu_param [H] and c = mu = 0.1 + softplus(mu_param).
__device__ __forceinline__ float prior_precision(const float* prec0, int prec_mode, int b, int h, int H, int K,
                                                int i) {
  if (prec_mode == 1) return prec0[((int64_t)b * H + h) * K + i];
  return prec_mode == 2 ? 0.1f + softplusf(prec0[h]) : prec0[h];
}

// grid (B*H), block K: per channel, the chunk maps in groups of 8 with the next group's loads in
// flight while the current group is applied.
__global__ __launch_bounds__(256) void diag_gain_carry_v_kernel(const float4* __restrict__ maps,
                                                                const float* __restrict__ prec0, int prec_mode, int H,
                                                                int K, int NT, float* __restrict__ carry,
                                                                float* __restrict__ final_prec) {
  const int bh = blockIdx.x, b = bh / H, h = bh % H, i = threadIdx.x;
  if (i >= K) return;
  float p = 1.f / prior_precision(prec0, prec_mode, b, h, H, K, i);
  const int64_t cb = (int64_t)bh * NT;
  float4 cur[8], nxt[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) cur[u] = maps[(cb + min(u, NT - 1)) * K + i];
  for (int n0 = 0; n0 < NT; n0 += 8) {
#pragma unroll
    for (int u = 0; u < 8; ++u) nxt[u] = maps[(cb + min(n0 + 8 + u, NT - 1)) * K + i];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (n0 + u >= NT) break;
      carry[(cb + n0 + u) * K + i] = p;
      p = (cur[u].x * p + cur[u].y) / (cur[u].z * p + cur[u].w);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) cur[u] = nxt[u];
  }
  if (final_prec) final_prec[((int64_t)b * H + h) * K + i] = 1.f / p;
}

__global__ __launch_bounds__(256) void diag_gain_emit_v_kernel(const float* __restrict__ k, const float* __restrict__ alpha,
                                                               const float* __restrict__ omega,
                                                               const float* __restrict__ r,
                                                               const float* __restrict__ carry, int B, int T, int H,
                                                               int K, int NT, float s, float* __restrict__ kappa,
                                                               float* __restrict__ p_prev, float* __restrict__ Dsave) {
  constexpr int NB = 4;
  const GainTile g = gain_tile(B, T, H, K, NT);
  if (!g.ok) return;
  const int tpt = K / kCPT;
  float p[kCPT];
  ldcf(carry + (((int64_t)g.b * H + g.h) * NT + g.nt) * K + g.i0, p);
  for (int t = g.t0; t < g.t1; t += NB) {
    float kt[NB][kCPT], al[NB][kCPT], wt[NB][kCPT], rt[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int64_t row = gain_row(g, T, H, min(t + u, g.t1 - 1));
      ldcf(k + row * K + g.i0, kt[u]);
      ldcf(alpha + row * K + g.i0, al[u]);
      ldcf(omega + row * K + g.i0, wt[u]);
      rt[u] = r[row];
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      if (t + u >= g.t1) break;
      const int64_t row = gain_row(g, T, H, t + u);
      const float ir = 1.f / rt[u];
      float num[kCPT], sq = 0.f;
      if (p_prev) stcf(p_prev + row * K + g.i0, p);
#pragma unroll
      for (int j = 0; j < kCPT; ++j) {
        const float ph = al[u][j] * al[u][j] * p[j] + wt[u][j];
        num[j] = ph * kt[u][j];
        sq += num[j] * kt[u][j];
        p[j] = ph / (1.f + s * kt[u][j] * kt[u][j] * ir * ph);
      }
      const float D = rt[u] + tile_sum(sq, tpt), iD = 1.f / D;
#pragma unroll
      for (int j = 0; j < kCPT; ++j) num[j] *= iD;
      stcf(kappa + row * K + g.i0, num);
      if (Dsave && g.sub == 0) Dsave[row] = D;
    }
  }
}

__global__ __launch_bounds__(256) void diag_gain_bwd_map_v_kernel(
    const float* __restrict__ k, const float* __restrict__ alpha, const float* __restrict__ omega,
    const float* __restrict__ r, const float* __restrict__ dkappa, const float* __restrict__ p_prev,
    const float* __restrict__ Dsave, int B, int T, int H, int K, int NT, float s, float* __restrict__ ab,
    float* __restrict__ Gsave) {
  constexpr int NB = 2;
  const GainTile g = gain_tile(B, T, H, K, NT);
  if (!g.ok) return;
  const int tpt = K / kCPT;
  float Aacc[kCPT], Bacc[kCPT];
#pragma unroll
  for (int j = 0; j < kCPT; ++j) Aacc[j] = 1.f, Bacc[j] = 0.f;
  for (int t = g.t1 - 1; t >= g.t0; t -= NB) {
    float kt[NB][kCPT], al[NB][kCPT], wt[NB][kCPT], pv[NB][kCPT], dk_[NB][kCPT], Dv[NB], rv[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int64_t row = gain_row(g, T, H, max(t - u, g.t0));
      ldcf(k + row * K + g.i0, kt[u]);
      ldcf(alpha + row * K + g.i0, al[u]);
      ldcf(omega + row * K + g.i0, wt[u]);
      ldcf(p_prev + row * K + g.i0, pv[u]);
      ldcf(dkappa + row * K + g.i0, dk_[u]);
      Dv[u] = Dsave[row];
      rv[u] = r[row];
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      if (t - u < g.t0) break;
      const float iD = 1.f / Dv[u], ir = 1.f / rv[u];
      float ph[kCPT], gp = 0.f;
#pragma unroll
      for (int j = 0; j < kCPT; ++j) {
        ph[j] = al[u][j] * al[u][j] * pv[u][j] + wt[u][j];
        gp += dk_[u][j] * ph[j] * kt[u][j];
      }
      const float G = tile_sum(gp, tpt) * iD;
#pragma unroll
      for (int j = 0; j < kCPT; ++j) {
        const float a2 = al[u][j] * al[u][j];
        const float hh = 1.f + s * kt[u][j] * kt[u][j] * ir * ph[j];
        const float pbar = dk_[u][j] * kt[u][j] * iD - kt[u][j] * kt[u][j] * G * iD;
        const float At = a2 / (hh * hh);
        Bacc[j] = At * Bacc[j] + a2 * pbar;
        Aacc[j] = At * Aacc[j];
      }
      if (Gsave && g.sub == 0) Gsave[gain_row(g, T, H, t - u)] = G;
    }
  }
  float4* dst = reinterpret_cast<float4*>(ab + ((((int64_t)g.b * H + g.h) * NT + g.nt) * K + g.i0) * 2);
#pragma unroll
  for (int q = 0; q < kCPT / 2; ++q) dst[q] = float4{Aacc[2 * q], Bacc[2 * q], Aacc[2 * q + 1], Bacc[2 * q + 1]};
}

__global__ __launch_bounds__(256) void diag_gain_bwd_carry_v_kernel(const float2* __restrict__ ab,
                                                                    const float* __restrict__ d_final_prec,
                                                                    const float* __restrict__ final_prec, int H,
                                                                    int K, int NT, float* __restrict__ carry) {
  const int bh = blockIdx.x, i = threadIdx.x;
  if (i >= K) return;
  float lam = 0.f;
  if (d_final_prec) {
    const float c = final_prec[(int64_t)bh * K + i];
    lam = -d_final_prec[(int64_t)bh * K + i] * c * c;
  }
  const int64_t cb = (int64_t)bh * NT;
  float2 cur[8], nxt[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) cur[u] = ab[(cb + max(NT - 1 - u, 0)) * K + i];
  for (int n1 = NT - 1; n1 >= 0; n1 -= 8) {
#pragma unroll
    for (int u = 0; u < 8; ++u) nxt[u] = ab[(cb + max(n1 - 8 - u, 0)) * K + i];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (n1 - u < 0) break;
      carry[(cb + n1 - u) * K + i] = lam;
      lam = cur[u].x * lam + cur[u].y;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) cur[u] = nxt[u];
  }
}

// Two-level carries for long streams.  A (b, h) stream of NT chunk maps per channel is cut into
// groups of kCarryGroup chunks: the groups' composite maps are formed in parallel (group_map), and every
// group then carries the stream's start value through the composites before it and replays its own chunk
// maps from there (group_fill), so no launch runs the serial carry over the composites.  The serial depth
// drops from NT to NG + 2 kCarryGroup steps.
// Forward maps are 2x2 Mobius maps on p (composed with max-abs renormalisation); backward maps are
// affine, lambda <- A lambda + B, applied from the last chunk down.
constexpr int kCarryGroup = 32;

// grid (B*H, NG), block K: composite of chunks [g G, min(NT, (g+1) G)) per channel
__global__ __launch_bounds__(256) void diag_gain_group_map_kernel(const float4* __restrict__ maps, int K, int NT,
                                                                  int NG, float4* __restrict__ gmaps) {
  const int bh = blockIdx.x, gi = blockIdx.y, i = threadIdx.x;
  if (i >= K) return;
  const int64_t cb = (int64_t)bh * NT;
  const int n0 = gi * kCarryGroup, n1 = min(NT, n0 + kCarryGroup);
  Map2 M{1.f, 0.f, 0.f, 1.f};
#pragma unroll 8
  for (int n = n0; n < n1; ++n) {
    const float4 m = maps[(cb + n) * K + i];
    M = map_mul(Map2{m.x, m.y, m.z, m.w}, M);
  }
  gmaps[((int64_t)bh * NG + gi) * K + i] = float4{M.m0, M.m1, M.m2, M.m3};
}
// grid (B*H, NG), block K: per-chunk carries (p entering each chunk) of group g.  Its start value is the
// prior's precision carried through the composites of groups 0 .. g-1, which each workgroup applies itself
// in order with the serial carry's arithmetic (diag_gain_carry_v_kernel over the composites gives the same
// values); the last group's workgroup also writes the final precision from its own composite.
__global__ __launch_bounds__(256) void diag_gain_group_fill_kernel(const float4* __restrict__ maps,
                                                                   const float4* __restrict__ gmaps,
                                                                   const float* __restrict__ prec0, int prec_mode,
                                                                   int H, int K, int NT, int NG,
                                                                   float* __restrict__ carry,
                                                                   float* __restrict__ final_prec) {
  const int bh = blockIdx.x, gi = blockIdx.y, i = threadIdx.x;
  if (i >= K) return;
  const int64_t cb = (int64_t)bh * NT;
  const int n0 = gi * kCarryGroup, n1 = min(NT, n0 + kCarryGroup);
  float p = 1.f / prior_precision(prec0, prec_mode, bh / H, bh % H, H, K, i);
  const float4* gm = gmaps + (int64_t)bh * NG * K + i;
#pragma unroll 8
  for (int g = 0; g < gi; ++g) {
    const float4 m = gm[(int64_t)g * K];
    p = (m.x * p + m.y) / (m.z * p + m.w);
  }
  if (final_prec && gi == NG - 1) {
    const float4 m = gm[(int64_t)gi * K];
    const float pf = (m.x * p + m.y) / (m.z * p + m.w);
    final_prec[(int64_t)bh * K + i] = 1.f / pf;
  }
#pragma unroll 8
  for (int n = n0; n < n1; ++n) {
    const float4 m = maps[(cb + n) * K + i];
    carry[(cb + n) * K + i] = p;
    p = (m.x * p + m.y) / (m.z * p + m.w);
  }
}
// grid (B*H, NG), block K: composite (A, B) of group g's reverse affine maps, last chunk first
__global__ __launch_bounds__(256) void diag_gain_bwd_group_map_kernel(const float2* __restrict__ ab, int K, int NT,
                                                                      int NG, float2* __restrict__ gab) {
  const int bh = blockIdx.x, gi = blockIdx.y, i = threadIdx.x;
  if (i >= K) return;
  const int64_t cb = (int64_t)bh * NT;
  const int n0 = gi * kCarryGroup, n1 = min(NT, n0 + kCarryGroup);
  float A = 1.f, Bc = 0.f;
#pragma unroll 8
  for (int n = n1 - 1; n >= n0; --n) {
    const float2 m = ab[(cb + n) * K + i];
    Bc = m.x * Bc + m.y;
    A = m.x * A;
  }
  gab[((int64_t)bh * NG + gi) * K + i] = float2{A, Bc};
}
// grid (B*H, NG), block K: per-chunk adjoint carries of group g from lambda leaving the group: the final
// precision's cotangent carried through the composites of groups NG-1 .. g+1, which each workgroup applies
// itself in that order with the serial carry's arithmetic (diag_gain_bwd_carry_v_kernel over the composites
// gives the same values).
__global__ __launch_bounds__(256) void diag_gain_bwd_group_fill_kernel(const float2* __restrict__ ab,
                                                                       const float2* __restrict__ gab,
                                                                       const float* __restrict__ d_final_prec,
                                                                       const float* __restrict__ final_prec, int K,
                                                                       int NT, int NG, float* __restrict__ carry) {
  const int bh = blockIdx.x, gi = blockIdx.y, i = threadIdx.x;
  if (i >= K) return;
  const int64_t cb = (int64_t)bh * NT;
  const int n0 = gi * kCarryGroup, n1 = min(NT, n0 + kCarryGroup);
  float lam = 0.f;
  if (d_final_prec) {
    const float c = final_prec[(int64_t)bh * K + i];
    lam = -d_final_prec[(int64_t)bh * K + i] * c * c;
  }
  const float2* gm = gab + (int64_t)bh * NG * K + i;
#pragma unroll 8
  for (int g = NG - 1; g > gi; --g) {
    const float2 m = gm[(int64_t)g * K];
    lam = m.x * lam + m.y;
  }
#pragma unroll 8
  for (int n = n1 - 1; n >= n0; --n) {
    const float2 m = ab[(cb + n) * K + i];
    carry[(cb + n) * K + i] = lam;
    lam = m.x * lam + m.y;
  }
}

__global__ __launch_bounds__(256) void diag_gain_bwd_emit_v_kernel(
    const float* __restrict__ k, const float* __restrict__ alpha, const float* __restrict__ omega,
    const float* __restrict__ r, const float* __restrict__ dkappa, const float* __restrict__ p_prev,
    const float* __restrict__ Dsave, const float* __restrict__ Gsave, const float* __restrict__ carry,
    const bf16_t* __restrict__ omega_raw, const bf16_t* __restrict__ r_raw, const float* __restrict__ prec0,
    int prec_mode, int B, int T, int H, int K, int NT, float s, float* __restrict__ dk, float* __restrict__ dalpha,
    bf16_t* __restrict__ domega_raw, bf16_t* __restrict__ dr_raw, float* __restrict__ dprec_part) {
  constexpr int NB = 2;
  const GainTile g = gain_tile(B, T, H, K, NT);
  if (!g.ok) return;
  const int tpt = K / kCPT;
  float lam[kCPT];
  ldcf(carry + (((int64_t)g.b * H + g.h) * NT + g.nt) * K + g.i0, lam);
  for (int t = g.t1 - 1; t >= g.t0; t -= NB) {
    float kt[NB][kCPT], al[NB][kCPT], wt[NB][kCPT], pv[NB][kCPT], dk_[NB][kCPT], Dv[NB], Gv[NB], rv[NB];
    float ow[NB][kCPT];
    bf16_t rr[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int64_t row = gain_row(g, T, H, max(t - u, g.t0));
      ldcf(k + row * K + g.i0, kt[u]);
      ldcf(alpha + row * K + g.i0, al[u]);
      ldcf(omega + row * K + g.i0, wt[u]);
      ldcf(p_prev + row * K + g.i0, pv[u]);
      ldcf(dkappa + row * K + g.i0, dk_[u]);
      ldc_bf16(omega_raw + row * K + g.i0, ow[u]);
      Dv[u] = Dsave[row];
      Gv[u] = Gsave[row];
      rv[u] = r[row];
      rr[u] = r_raw[row];
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      if (t - u < g.t0) break;
      const int64_t row = gain_row(g, T, H, t - u);
      const float* oraw = ow[u];
      float dko[kCPT], dao[kCPT], dwo[kCPT];
      const float G = Gv[u], iD = 1.f / Dv[u], ir = 1.f / rv[u];
      float urr = 0.f;
#pragma unroll
      for (int j = 0; j < kCPT; ++j) {
        const float a2 = al[u][j] * al[u][j];
        const float ph = a2 * pv[u][j] + wt[u][j];
        const float uu = s * kt[u][j] * kt[u][j] * ir;
        const float hh = 1.f + uu * ph, ihh = 1.f / hh;
        const float pnext = ph * ihh;
        const float pbar = dk_[u][j] * kt[u][j] * iD - kt[u][j] * kt[u][j] * G * iD + lam[j] * ihh * ihh;
        const float ubar = -lam[j] * pnext * pnext;
        dko[j] = dk_[u][j] * ph * iD - 2.f * ph * kt[u][j] * G * iD + ubar * (2.f * s * kt[u][j] * ir);
        dao[j] = 2.f * al[u][j] * pv[u][j] * pbar;
        dwo[j] = pbar * sigmoidf(oraw[j]);
        urr += ubar * (-s * kt[u][j] * kt[u][j] * ir * ir);
        lam[j] = a2 * pbar;
      }
      stcf(dk + row * K + g.i0, dko);
      stcf(dalpha + row * K + g.i0, dao);
      stc_bf16(domega_raw + row * K + g.i0, dwo);
      const float utot = tile_sum(urr, tpt);
      if (g.sub == 0) dr_raw[row] = f2bf((-G * iD + utot) * sigmoidf(bf2f(rr[u])));
    }
  }
  if (g.nt == 0 && dprec_part) {
    // lam holds dL/dp_{-1}; p_{-1} = 1/c  ->  dL/dc = -lam p^2
    float cN[kCPT], part = 0.f;
    if (prec_mode == 1) ldcf(prec0 + ((int64_t)g.b * H + g.h) * K + g.i0, cN);
#pragma unroll
    for (int j = 0; j < kCPT; ++j) {
      const float c = prec_mode == 0 ? prec0[g.h] : cN[j];
      const float p0 = 1.f / c;
      cN[j] = -lam[j] * p0 * p0;
      part += cN[j];
    }
    if (prec_mode == 1) {
      stcf(dprec_part + ((int64_t)g.b * H + g.h) * K + g.i0, cN);
    } else {
      part = tile_sum(part, tpt);
      if (g.sub == 0) dprec_part[(int64_t)g.b * H + g.h] = part;
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

// ----------------------------------------------------------------------------
// Fused diag frontend + gain ("front").  The layer composition (reference lit_gpt/diag_kdn.py:315-345)
// runs the q/k normalisation, the retention frontend and the vector gain back to back, and the
// frontend's alpha, omega, r and the normalised fp32 key feed only the gain.  Here the gain's map and
// emit passes recompute them per token from the raw bf16 logits and the raw key with its row norm,
// using the standalone kernels' own operations, and the emit pass also writes the chunk-local base-2
// log-decay prefix g_cumsum.  So alpha, omega and the fp32 key are never written or read back.
// The backward replays each 16-token tile's precision from the tile's saved entry value (the
// forward's carry, B*H*NV*K floats) instead of reading a stored p_prev [B,T,H,K], and finishes
// with the raw-logit, decay-parameter and key-normalisation VJPs in the same pass.
// Tiles are the vectorised gain's: (b, h, 16 tokens) x K channels, kCPT channels per thread.
// ----------------------------------------------------------------------------
// Addresses in the fused kernels are 32-bit element offsets from a kernel-argument base (the
// scalar-base + vector-offset form, one offset register per access instead of a 64-bit address
// pair); the host splits a launch over the batch so every array stays below 2^30 elements.
template <typename T> __device__ __forceinline__ T* off32(T* base, uint32_t elem) {
  return reinterpret_cast<T*>(reinterpret_cast<char*>(base) + elem * (uint32_t)sizeof(T));
}
template <typename T> __device__ __forceinline__ const T* off32(const T* base, uint32_t elem) {
  return reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) + elem * (uint32_t)sizeof(T));
}
__device__ __forceinline__ uint32_t front_row(const GainTile& g, int T, int H, int t) {
  return ((uint32_t)g.b * (uint32_t)T + (uint32_t)t) * (uint32_t)H + (uint32_t)g.h;
}
constexpr float kFloorLog = -13.815510557964274f;  // log(1e-6): the memory path's alpha floor
constexpr int kPairs = kVecChunk / 2;  // token pairs of a tile (the saved precisions: one per even token)
static_assert(kCPT == 4, "a thread's saved precisions are one float4");

template <typename TX> __device__ __forceinline__ void ldk4(const TX* p, float* f);
template <> __device__ __forceinline__ void ldk4<float>(const float* p, float* f) { ldcf(p, f); }
template <> __device__ __forceinline__ void ldk4<bf16_t>(const bf16_t* p, float* f) { ldc_bf16(p, f); }
template <typename TX> __device__ __forceinline__ void stk4(TX* p, const float* f);
template <> __device__ __forceinline__ void stk4<float>(float* p, const float* f) { stcf(p, f); }
template <> __device__ __forceinline__ void stk4<bf16_t>(bf16_t* p, const float* f) { stc_bf16(p, f); }

template <typename TX>
struct FrontArgs {
  const TX* k;           // key before normalisation [B,T,H,K]
  const float* knorm;    // its row norms ||k|| [B,T,H]
  const bf16_t* f;       // retention logits [B,T,H,K]
  const bf16_t* z;       // omega logits [B,T,H,K]
  const bf16_t* y;       // r logits [B,T,H]
  const float* A_log;    // [H]
  const float* dt_bias;  // [H,K]
  int B, T, H, K, NV;    // NV 16-token tiles per (b, h) stream
  int tpc;               // tiles per decay chunk (chunk / 16)
  float s;               // info scale
};

// Raw inputs of one token for one thread's kCPT channels.  bf16 values stay packed until use, which
// keeps the loads of two tokens in flight within the register budget.
struct Bf4 {
  uint2 v;
};
__device__ __forceinline__ Bf4 ldbf4(const bf16_t* p) { return Bf4{*reinterpret_cast<const uint2*>(p)}; }
__device__ __forceinline__ float bfj(const Bf4& b, int j) {
  const uint32_t w = j < 2 ? b.v.x : b.v.y;
  return __uint_as_float((j & 1) ? (w & 0xffff0000u) : (w << 16));
}
template <typename TX> struct K4;
template <> struct K4<bf16_t> {
  Bf4 b;
  __device__ __forceinline__ void load(const bf16_t* p) { b = ldbf4(p); }
  __device__ __forceinline__ float operator[](int j) const { return bfj(b, j); }
};
template <> struct K4<float> {
  float4 v;
  __device__ __forceinline__ void load(const float* p) { v = *reinterpret_cast<const float4*>(p); }
  __device__ __forceinline__ float operator[](int j) const { return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w; }
};
template <typename TX>
struct FrontRaw {
  K4<TX> k;
  Bf4 f, z;
  float kn, y;
};
template <typename TX>
__device__ __forceinline__ void front_load(const FrontArgs<TX>& a, uint32_t row, int i0, FrontRaw<TX>& r) {
  const uint32_t e = row * (uint32_t)a.K + (uint32_t)i0;
  r.k.load(off32(a.k, e));
  r.f = ldbf4(off32(a.f, e));
  r.z = ldbf4(off32(a.z, e));
  r.kn = *off32(a.knorm, row);
  r.y = bf2f(*off32(a.y, row));
}
// The gain's per-token inputs for one thread's kCPT channels: kt = k / max(||k||, 1e-12),
// ell = -e^A softplus(f + dt_bias), alpha = e^ell, omega = softplus(z), 1/r with r = 0.01 + softplus(y).
// With BWD also the sigmoids the backward needs (sigma(f + dt_bias), sigma(z), sigma(y)), each from
// the exponential its softplus already took.  Reciprocals are the hardware v_rcp_f32 (1 ulp): these
// passes are bound by vector-ALU issue, and an IEEE division costs ten instructions.
struct FrontTok {
  float kt[kCPT], al[kCPT], wt[kCPT], ell[kCPT];
  float r, ir;
};
struct FrontSig {
  float f[kCPT], z[kCPT];
  float y;
};
template <bool BWD, typename TX>
__device__ __forceinline__ void front_tok(const FrontRaw<TX>& r, float rate, const float* bias, FrontTok& o,
                                          FrontSig& sg) {
  const float ik = frcp(fmaxf(r.kn, 1e-12f));
#pragma unroll
  for (int j = 0; j < kCPT; ++j) {
    o.kt[j] = r.k[j] * ik;
    float spf;
    if (BWD) {
      fsoftplus_sigmoid(bfj(r.f, j) + bias[j], spf, sg.f[j]);
      fsoftplus_sigmoid(bfj(r.z, j), o.wt[j], sg.z[j]);
    } else {
      spf = fsoftplus(bfj(r.f, j) + bias[j]);
      o.wt[j] = fsoftplus(bfj(r.z, j));
    }
    o.ell[j] = -rate * spf;
    o.al[j] = fexp(o.ell[j]);
  }
  float spy;
  if (BWD) {
    fsoftplus_sigmoid(r.y, spy, sg.y);
  } else {
    spy = fsoftplus(r.y);
  }
  o.r = 0.01f + spy;
  o.ir = frcp(o.r);
}
// the memory path's clamped log-decay (NaN propagates)
__device__ __forceinline__ float ell_mem(float ell, float al) {
  const bool floor = al < 1e-6f;  // false for NaN, which propagates
  return floor ? kFloorLog : ell;
}
// p entering the next token: p' = p_hat / (1 + s k^2 / r p_hat), p_hat = alpha^2 p + omega
__device__ __forceinline__ void front_step(const float* pin, const FrontTok& t, float s, float* pout) {
#pragma unroll
  for (int j = 0; j < kCPT; ++j) {
    const float ph = t.al[j] * t.al[j] * pin[j] + t.wt[j];
    pout[j] = ph * frcp(1.f + s * t.kt[j] * t.kt[j] * t.ir * ph);
  }
}
// 2x2 product without renormalisation (entries are non-negative and the (2,2) entry of a product of
// token maps is >= 1, so four tokens stay far inside fp32 range before the renormalisation)
__device__ __forceinline__ Map2 map_mul_raw(const Map2& a, const Map2& b) {
  return Map2{a.m0 * b.m0 + a.m1 * b.m2, a.m0 * b.m1 + a.m1 * b.m3, a.m2 * b.m0 + a.m3 * b.m2,
              a.m2 * b.m1 + a.m3 * b.m3};
}
__device__ __forceinline__ void map_renorm(Map2& c) {
  const float s = fmaxf(fmaxf(fabsf(c.m0), fabsf(c.m1)), fmaxf(fabsf(c.m2), fabsf(c.m3)));
  const float inv = frcp(fmaxf(s, 1e-30f));
  c.m0 *= inv, c.m1 *= inv, c.m2 *= inv, c.m3 *= inv;
}

// Forward map: per channel the tile's composite Mobius map, and the tile's sum of clamped log-decays.
template <typename TX>
// 8 workgroups (waves per SIMD) per CU: the pass hides its loads' latency with waves, 2 tokens in flight each
__global__ __launch_bounds__(256, 8) void diag_front_map_kernel(FrontArgs<TX> a, float* __restrict__ maps,
                                                             float* __restrict__ tsum) {
  constexpr int NB = 2;
  const GainTile g = gain_tile(a.B, a.T, a.H, a.K, a.NV);
  if (!g.ok) return;
  const float rate = __expf(a.A_log[g.h]);
  float bias[kCPT], es[kCPT];
  ldcf(a.dt_bias + g.h * a.K + g.i0, bias);
  Map2 M[kCPT];
#pragma unroll
  for (int j = 0; j < kCPT; ++j) M[j] = Map2{1.f, 0.f, 0.f, 1.f}, es[j] = 0.f;
  // one token's step: its log-decay into the tile sum, its map onto the composite
  auto step = [&](const FrontRaw<TX>& raw) {
    FrontTok tk;
    FrontSig unused;
    front_tok<false>(raw, rate, bias, tk, unused);
#pragma unroll
    for (int j = 0; j < kCPT; ++j) {
      es[j] += ell_mem(tk.ell[j], tk.al[j]);
      const float a2 = tk.al[j] * tk.al[j], uu = a.s * tk.kt[j] * tk.kt[j] * tk.ir;
      M[j] = map_mul_raw(Map2{a2, tk.wt[j], uu * a2, 1.f + uu * tk.wt[j]}, M[j]);
    }
  };
  for (int t = g.t0; t < g.t1; t += NB) {
    FrontRaw<TX> raw[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) front_load(a, front_row(g, a.T, a.H, min(t + u, g.t1 - 1)), g.i0, raw[u]);
    if (t + NB <= g.t1) {
      // every token of the group is in the tile: no per-token condition, so the compiler keeps the
      // NB tokens' loads in flight together instead of sinking each into its token's branch
#pragma unroll
      for (int u = 0; u < NB; ++u) step(raw[u]);
    } else {
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        if (t + u >= g.t1) break;
        step(raw[u]);
      }
    }
#pragma unroll
    for (int j = 0; j < kCPT; ++j) map_renorm(M[j]);
  }
  const uint32_t tb = (((uint32_t)g.b * a.H + g.h) * a.NV + g.nt) * (uint32_t)a.K + g.i0;
  float4* dst = reinterpret_cast<float4*>(off32(maps, tb * 4u));
#pragma unroll
  for (int j = 0; j < kCPT; ++j) dst[j] = float4{M[j].m0, M[j].m1, M[j].m2, M[j].m3};
  stcf(off32(tsum, tb), es);
}

// Forward emit: kappa and g_cumsum per token from the tile's entry precision.  The decay prefix
// starts from the sum of the earlier tiles of the same decay chunk.
template <typename TX>
__global__ __launch_bounds__(256) void diag_front_emit_kernel(FrontArgs<TX> a, const float* __restrict__ carry,
                                                              const float* __restrict__ tsum,
                                                              float* __restrict__ g_cumsum,
                                                              float* __restrict__ kappa, float* __restrict__ pe) {
  constexpr int NB = 4;
  const GainTile g = gain_tile(a.B, a.T, a.H, a.K, a.NV);
  if (!g.ok) return;
  const int tpt = a.K / kCPT;
  const float rate = __expf(a.A_log[g.h]);
  float bias[kCPT], p[kCPT], acc[kCPT];
  ldcf(a.dt_bias + g.h * a.K + g.i0, bias);
  const uint32_t sb = ((uint32_t)g.b * a.H + g.h) * a.NV;
  ldcf(off32(carry, (sb + g.nt) * (uint32_t)a.K + g.i0), p);
#pragma unroll
  for (int j = 0; j < kCPT; ++j) acc[j] = 0.f;
  for (int n = g.nt - g.nt % a.tpc; n < g.nt; ++n) {
    float e[kCPT];
    ldcf(off32(tsum, (sb + n) * (uint32_t)a.K + g.i0), e);
#pragma unroll
    for (int j = 0; j < kCPT; ++j) acc[j] += e[j];
  }
  for (int t = g.t0; t < g.t1; t += NB) {
    FrontRaw<TX> raw[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) front_load(a, front_row(g, a.T, a.H, min(t + u, g.t1 - 1)), g.i0, raw[u]);
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      if (t + u >= g.t1) break;
      const uint32_t row = front_row(g, a.T, a.H, t + u);
      if (pe && ((t + u - g.t0) & 1) == 0)  // the precision entering an even token, for the backward
        *reinterpret_cast<float4*>(off32(pe, ((sb + g.nt) * kPairs + ((t + u - g.t0) >> 1)) * (uint32_t)a.K + g.i0)) =
            float4{p[0], p[1], p[2], p[3]};
      FrontTok tk;
      FrontSig unused;
      front_tok<false>(raw[u], rate, bias, tk, unused);
      float num[kCPT], gc[kCPT], sq = 0.f;
#pragma unroll
      for (int j = 0; j < kCPT; ++j) {
        acc[j] += ell_mem(tk.ell[j], tk.al[j]);
        gc[j] = acc[j] * KDN_LOG2E;
        const float ph = tk.al[j] * tk.al[j] * p[j] + tk.wt[j];
        num[j] = ph * tk.kt[j];
        sq += num[j] * tk.kt[j];
        p[j] = ph * frcp(1.f + a.s * tk.kt[j] * tk.kt[j] * tk.ir * ph);
      }
      const float iD = frcp(tk.r + tile_sum(sq, tpt));
#pragma unroll
      for (int j = 0; j < kCPT; ++j) num[j] *= iD;
      stcf(off32(kappa, row * (uint32_t)a.K + (uint32_t)g.i0), num);
      stcf(off32(g_cumsum, row * (uint32_t)a.K + (uint32_t)g.i0), gc);
    }
  }
}

// The backward passes need p_{t-1}, the precision entering each token, in reverse token order.  The
// forward's emit pass saved the precision entering every even token of each tile (pe); the reverse pass
// takes the tokens in pairs (2q + 1, 2q), loads the pair's saved value with the pair's other inputs
// (float4 per thread) and re-derives the odd token's entry value with one forward step of token 2q,
// whose inputs it computes anyway.  (Staged in LDS for the whole tile, the values took 32 KB per
// workgroup, which held the passes to five workgroups per CU.)
__device__ __forceinline__ float4 f4(const float* x) { return float4{x[0], x[1], x[2], x[3]}; }
__device__ __forceinline__ void unf4(float4 v, float* x) { x[0] = v.x, x[1] = v.y, x[2] = v.z, x[3] = v.w; }
// this thread's saved entry precisions of token pair q of its tile
__device__ __forceinline__ float4 front_pe(const float* __restrict__ pe, const GainTile& g, int H, int NV, int K, int q) {
  const uint32_t tile = ((uint32_t)g.b * H + g.h) * NV + g.nt;
  return *reinterpret_cast<const float4*>(off32(pe, (tile * kPairs + q) * (uint32_t)K + g.i0));
}

// Backward map (reverse over the tile): the affine adjoint map (A, B) per channel, the per-token
// gain denominator D_t and G_t = sum_i dkappa_i p_hat_i k_i / D_t (saved for the emit pass), and the
// tile's sum of the g_cumsum cotangent (for the emit pass's chunk-suffix sums).
template <typename TX>
__global__ __launch_bounds__(256) void diag_front_bwd_map_kernel(FrontArgs<TX> a, const float* __restrict__ pe,
                                                                 const float* __restrict__ dkappa,
                                                                 const float* __restrict__ dG, float* __restrict__ ab,
                                                                 float* __restrict__ tdg, float* __restrict__ Gsave,
                                                                 float* __restrict__ Dsave) {
  const GainTile g = gain_tile(a.B, a.T, a.H, a.K, a.NV);
  if (!g.ok) return;
  const int tpt = a.K / kCPT, L = g.t1 - g.t0;
  const float rate = __expf(a.A_log[g.h]);
  float bias[kCPT];
  ldcf(a.dt_bias + g.h * a.K + g.i0, bias);
  float Aacc[kCPT], Bacc[kCPT], sg[kCPT];
#pragma unroll
  for (int j = 0; j < kCPT; ++j) Aacc[j] = 1.f, Bacc[j] = 0.f, sg[j] = 0.f;
#pragma unroll 1
  for (int q = (L - 1) >> 1; q >= 0; --q) {
    FrontRaw<TX> raw[2];
    float dk_[2][kCPT], dg_[2][kCPT];
    const float4 pe_q = front_pe(pe, g, a.H, a.NV, a.K, q);
#pragma unroll
    for (int u = 0; u < 2; ++u) {  // u = 0: token 2q + 1, u = 1: token 2q
      const uint32_t row = front_row(g, a.T, a.H, g.t0 + min(2 * q + 1 - u, L - 1));
      front_load(a, row, g.i0, raw[u]);
      ldcf(off32(dkappa, row * (uint32_t)a.K + (uint32_t)g.i0), dk_[u]);
      ldcf(off32(dG, row * (uint32_t)a.K + (uint32_t)g.i0), dg_[u]);
    }
    FrontTok tk[2];
    FrontSig unused;
    float pp[2][kCPT];
#pragma unroll
    for (int u = 0; u < 2; ++u) front_tok<false>(raw[u], rate, bias, tk[u], unused);
    unf4(pe_q, pp[1]);
    front_step(pp[1], tk[1], a.s, pp[0]);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int tt = 2 * q + 1 - u;
      if (tt < L) {
        float ph[kCPT], sq = 0.f, gp = 0.f;
#pragma unroll
        for (int j = 0; j < kCPT; ++j) {
          ph[j] = tk[u].al[j] * tk[u].al[j] * pp[u][j] + tk[u].wt[j];
          const float num = ph[j] * tk[u].kt[j];
          sq += num * tk[u].kt[j];
          gp += dk_[u][j] * num;
        }
        const float D = tk[u].r + tile_sum(sq, tpt), iD = frcp(D);
        const float G = tile_sum(gp, tpt) * iD;
#pragma unroll
        for (int j = 0; j < kCPT; ++j) {
          const float a2 = tk[u].al[j] * tk[u].al[j], k2 = tk[u].kt[j] * tk[u].kt[j];
          const float ihh = frcp(1.f + a.s * k2 * tk[u].ir * ph[j]);
          const float pbar = (dk_[u][j] * tk[u].kt[j] - k2 * G) * iD;
          const float At = a2 * ihh * ihh;
          Bacc[j] = At * Bacc[j] + a2 * pbar;
          Aacc[j] = At * Aacc[j];
          sg[j] += dg_[u][j];
        }
        if (g.sub == 0) {
          const uint32_t row = front_row(g, a.T, a.H, g.t0 + tt);
          *off32(Gsave, row) = G;
          *off32(Dsave, row) = D;
        }
      }
    }
  }
  const uint32_t tb = (((uint32_t)g.b * a.H + g.h) * a.NV + g.nt) * (uint32_t)a.K + g.i0;
  float4* dst = reinterpret_cast<float4*>(off32(ab, tb * 2u));
#pragma unroll
  for (int q = 0; q < kCPT / 2; ++q) dst[q] = float4{Aacc[2 * q], Bacc[2 * q], Aacc[2 * q + 1], Bacc[2 * q + 1]};
  stcf(off32(tdg, tb), sg);
}

// Backward emit (reverse over the tile): the gain adjoint from the carried lambda, then per token
//   d omega_raw = p_bar sigmoid(z), d r_raw (tile sum), d retention_raw from
//   d ell = [alpha >= 1e-6] (suffix sum of dG in the decay chunk) + d alpha * alpha,
// per-tile partials of dA_log (sum d ell * ell) and d dt_bias (sum d f), and the key VJP of
// k / max(||k||, 1e-12) applied to dk_gain + dk_memory (dk_memory nullable; dk nullable).
template <typename TX>
__global__ __launch_bounds__(256) void diag_front_bwd_emit_kernel(
    FrontArgs<TX> a, const float* __restrict__ pe, const float* __restrict__ lcarry,
    const float* __restrict__ dkappa, const float* __restrict__ dG, const float* __restrict__ tdg,
    const float* __restrict__ Gsave, const float* __restrict__ Dsave, const bf16_t* __restrict__ dk_mem,
    const float* __restrict__ prec0, int prec_mode, TX* __restrict__ dk, bf16_t* __restrict__ df,
    bf16_t* __restrict__ dz, bf16_t* __restrict__ dy, float* __restrict__ part_A, float* __restrict__ part_dt,
    float* __restrict__ dprec_part) {
  const GainTile g = gain_tile(a.B, a.T, a.H, a.K, a.NV);
  if (!g.ok) return;
  const int tpt = a.K / kCPT, L = g.t1 - g.t0;
  const float rate = __expf(a.A_log[g.h]);
  float bias[kCPT];
  ldcf(a.dt_bias + g.h * a.K + g.i0, bias);
  const uint32_t sb = ((uint32_t)g.b * a.H + g.h) * a.NV;
  float lam[kCPT], accg[kCPT], ddt[kCPT], dA = 0.f;
  ldcf(off32(lcarry, (sb + g.nt) * (uint32_t)a.K + g.i0), lam);
#pragma unroll
  for (int j = 0; j < kCPT; ++j) accg[j] = 0.f, ddt[j] = 0.f;
  const int n_end = min(a.NV, g.nt - g.nt % a.tpc + a.tpc);
  for (int n = g.nt + 1; n < n_end; ++n) {
    float e[kCPT];
    ldcf(off32(tdg, (sb + n) * (uint32_t)a.K + g.i0), e);
#pragma unroll
    for (int j = 0; j < kCPT; ++j) accg[j] += e[j];
  }
#pragma unroll 1
  for (int q = (L - 1) >> 1; q >= 0; --q) {
    FrontRaw<TX> raw[2];
    float dk_[2][kCPT], dg_[2][kCPT], Gv[2], Dv[2];
    Bf4 dkm[2];
    const float4 pe_q = front_pe(pe, g, a.H, a.NV, a.K, q);
#pragma unroll
    for (int u = 0; u < 2; ++u) {  // u = 0: token 2q + 1, u = 1: token 2q
      const uint32_t row = front_row(g, a.T, a.H, g.t0 + min(2 * q + 1 - u, L - 1));
      front_load(a, row, g.i0, raw[u]);
      ldcf(off32(dkappa, row * (uint32_t)a.K + (uint32_t)g.i0), dk_[u]);
      ldcf(off32(dG, row * (uint32_t)a.K + (uint32_t)g.i0), dg_[u]);
      dkm[u] = dk_mem ? ldbf4(off32(dk_mem, row * (uint32_t)a.K + (uint32_t)g.i0)) : Bf4{uint2{0u, 0u}};
      Gv[u] = *off32(Gsave, row);
      Dv[u] = *off32(Dsave, row);
    }
    FrontTok tk[2];
    FrontSig sgm[2];
    float pp[2][kCPT];
#pragma unroll
    for (int u = 0; u < 2; ++u) front_tok<true>(raw[u], rate, bias, tk[u], sgm[u]);
    unf4(pe_q, pp[1]);
    front_step(pp[1], tk[1], a.s, pp[0]);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int tt = 2 * q + 1 - u;
      if (tt < L) {
        const uint32_t row = front_row(g, a.T, a.H, g.t0 + tt);
        const FrontTok& t = tk[u];
        float dko[kCPT], dfo[kCPT], dwo[kCPT];
        const float G = Gv[u], iD = frcp(Dv[u]);
        float urr = 0.f;
#pragma unroll
        for (int j = 0; j < kCPT; ++j) {
          const float a2 = t.al[j] * t.al[j], k2 = t.kt[j] * t.kt[j];
          const float ph = a2 * pp[u][j] + t.wt[j];
          const float uu = a.s * k2 * t.ir;
          const float ihh = frcp(1.f + uu * ph);
          const float pnext = ph * ihh;
          const float pbar = (dk_[u][j] * t.kt[j] - k2 * G) * iD + lam[j] * ihh * ihh;
          const float ubar = -lam[j] * pnext * pnext;
          dko[j] = (dk_[u][j] - 2.f * t.kt[j] * G) * ph * iD + ubar * (2.f * a.s * t.kt[j] * t.ir);
          const float dao = 2.f * t.al[j] * pp[u][j] * pbar;
          dwo[j] = pbar * sgm[u].z[j];
          urr -= ubar * uu * t.ir;
          lam[j] = a2 * pbar;
          // retention frontend: alpha = exp(ell), ell = -e^A softplus(f + dt_bias)
          accg[j] += dg_[u][j];
          float dell = t.al[j] >= 1e-6f ? accg[j] : 0.f;
          dell += dao * t.al[j];
          dfo[j] = dell * (-rate) * sgm[u].f[j];
          dA += dell * t.ell[j];
          ddt[j] += dfo[j];
        }
        stc_bf16(off32(df, row * (uint32_t)a.K + (uint32_t)g.i0), dfo);
        stc_bf16(off32(dz, row * (uint32_t)a.K + (uint32_t)g.i0), dwo);
        const float utot = tile_sum(urr, tpt);
        if (g.sub == 0) *off32(dy, row) = f2bf((-G * iD + utot) * sgm[u].y);
        if (dk) {  // VJP of kt = k / max(||k||, 1e-12) applied to dk_gain + dk_memory
          float gk[kCPT], dot = 0.f;
#pragma unroll
          for (int j = 0; j < kCPT; ++j) {
            gk[j] = dko[j] + bfj(dkm[u], j);
            dot += t.kt[j] * gk[j];
          }
          dot = tile_sum(dot, tpt);
          const float id = frcp(fmaxf(raw[u].kn, 1e-12f));
          const bool clamped = !(raw[u].kn > 1e-12f);
#pragma unroll
          for (int j = 0; j < kCPT; ++j) gk[j] = clamped ? gk[j] * id : (gk[j] - t.kt[j] * dot) * id;
          stk4<TX>(off32(dk, row * (uint32_t)a.K + (uint32_t)g.i0), gk);
        }
      }
    }
  }
  const uint32_t P = (uint32_t)g.b * a.NV + g.nt;
  if (part_dt) stcf(off32(part_dt, (P * a.H + g.h) * (uint32_t)a.K + g.i0), ddt);
  dA = tile_sum(dA, tpt);
  if (part_A && g.sub == 0) *off32(part_A, P * a.H + g.h) = dA;
  if (g.nt == 0 && dprec_part) {  // lam holds dL/dp_{-1}; p_{-1} = 1/c  ->  dL/dc = -lam p^2
    float cN[kCPT], part = 0.f;
    if (prec_mode == 1) ldcf(prec0 + ((int64_t)g.b * a.H + g.h) * a.K + g.i0, cN);
    const float c_head = prec_mode == 1 ? 0.f : prior_precision(prec0, prec_mode, g.b, g.h, a.H, a.K, 0);
#pragma unroll
    for (int j = 0; j < kCPT; ++j) {
      const float c = prec_mode == 1 ? cN[j] : c_head;
      const float p0 = 1.f / c;
      cN[j] = -lam[j] * p0 * p0;
      part += cN[j];
    }
    if (prec_mode == 1) {
      stcf(dprec_part + ((int64_t)g.b * a.H + g.h) * a.K + g.i0, cN);
    } else {
      part = tile_sum(part, tpt);
      if (g.sub == 0) dprec_part[(int64_t)g.b * a.H + g.h] = part;
    }
  }
}

inline int cdiv(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }
// Fixed device workspace of kdn_iso_gain_fwd_noalloc (the per-chunk maps and carries of the iso gain),
// for callers that cannot allocate.  Each GPU the library runs on holds its own copy until the process
// ends.  In host code `scratch` names a host-side stand-in; the device address comes from
// hipGetSymbolAddress, taken once per device with that device current and kept in g_scratch_ptr.
static __device__ __align__(256) unsigned char scratch[KDN_NOALLOC_SCRATCH_BYTES];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's `scratch` (looked up on the first call per device).
int current_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return KDN_ERR_ARG;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (p == nullptr) return (int)hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

inline int gain_block(int K) { return ((K + 63) / 64) * 64; }
inline bool gain_vec_ok(int K) { return K % kCPT == 0 && 64 % (K / kCPT) == 0; }
inline bool aligned16(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" {

size_t kdn_iso_gain_workspace_size(int B, int T, int H) {
  const int64_t NC = cdiv(T, kIsoChunk);
  return (size_t)((int64_t)B * H * NC * 5) * sizeof(float);
}

int kdn_iso_gain_fwd(const float* a, const float* omega, const float* r, const float* initial_precision,
                     int prec_mode, int B, int T, int H, float posterior_scale, float* beta, float* p_prev,
                     float* final_precision, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (B < 0 || T < 0 || H <= 0 || H > 96 || !(posterior_scale > 0.f) || (prec_mode != 0 && prec_mode != 1))
    return KDN_ERR_ARG;
  if (B == 0 || T == 0) return 0;
  if (workspace_bytes < kdn_iso_gain_workspace_size(B, T, H)) return KDN_ERR_ARG;
  const int NC = cdiv(T, kIsoChunk);
  float4* maps = (float4*)workspace;
  const int unit = posterior_scale == 1.f ? 1 : 0;
  const size_t lds_map = (size_t)(3 * kIsoChunk * H + 4 * kIsoSub * H) * sizeof(float);
  hipLaunchKernelGGL(iso_gain_map_kernel, dim3(NC, B), dim3(256), lds_map, stream, a, omega, r, T, H, NC,
                     posterior_scale, maps);
  launch_iso_gain_emit(a, omega, r, maps, initial_precision, prec_mode, B, T, H, NC, posterior_scale, beta, p_prev,
                       final_precision, stream);
  KDN_CHECK_LAUNCH();
  return 0;
}

int kdn_iso_gain_fwd_noalloc(const float* a, const float* omega, const float* r, const float* initial_precision,
                             int prec_mode, int B, int T, int H, float posterior_scale, float* beta, float* p_prev,
                             float* final_precision, hipStream_t stream) {
  if (B < 0 || T < 0 || H <= 0 || H > 96 || !(posterior_scale > 0.f) || (prec_mode != 0 && prec_mode != 1))
    return KDN_ERR_ARG;
  if (B == 0 || T == 0) return 0;
  const size_t need = kdn_iso_gain_workspace_size(B, T, H);
  if (need > (size_t)KDN_NOALLOC_SCRATCH_BYTES) return KDN_ERR_ARG;
  if (stream != nullptr) {  // the fixed workspace used is the current device's: the stream must run there
    int sdev = -1, dev = -1;
    hipError_t e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess) return (int)e;
    e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (sdev != dev) return KDN_ERR_ARG;
  }
  void* ws = nullptr;
  const int rc = current_scratch(&ws);
  if (rc != 0) return rc;
  return kdn_iso_gain_fwd(a, omega, r, initial_precision, prec_mode, B, T, H, posterior_scale, beta, p_prev,
                          final_precision, ws, need, stream);
}

int kdn_iso_gain_bwd(const float* a, const float* omega, const float* r, const float* initial_precision,
                     int prec_mode, const float* dbeta, const float* p_prev, const float* final_precision,
                     const float* d_final_precision, int B, int T, int H, float posterior_scale, float* da,
                     float* domega, float* dr, float* d_initial_precision, void* workspace, size_t workspace_bytes,
                     hipStream_t stream) {
  if (B < 0 || T < 0 || H <= 0 || H > 96 || !(posterior_scale > 0.f) || (prec_mode != 0 && prec_mode != 1))
    return KDN_ERR_ARG;
  if (d_final_precision && !final_precision) return KDN_ERR_ARG;
  if (B == 0 || T == 0) return 0;
  if (workspace_bytes < kdn_iso_gain_workspace_size(B, T, H)) return KDN_ERR_ARG;
  const int NC = cdiv(T, kIsoChunk);
  float2* maps = (float2*)workspace;
  float* carry = (float*)(maps + (int64_t)B * H * NC);
  const int unit = posterior_scale == 1.f ? 1 : 0;
  const size_t lds_emit = (size_t)(8 * kIsoChunk * H + 2 * kIsoSub * H) * sizeof(float);
  const int GB = B < 16 ? B : 16;
  launch_iso_gain_bwd_map(a, omega, r, dbeta, p_prev, B, T, H, NC, posterior_scale, maps, stream);
  hipLaunchKernelGGL(iso_gain_bwd_carry_kernel, dim3(H), dim3(64 * GB), 0, stream, maps, initial_precision, prec_mode,
                     B, H, NC, final_precision, d_final_precision, carry, d_initial_precision);
  hipLaunchKernelGGL(iso_gain_bwd_emit_kernel, dim3(NC, B), dim3(256), lds_emit, stream, a, omega, r, dbeta, p_prev, T,
                     H, NC, posterior_scale, unit, carry, da, domega, dr);
  KDN_CHECK_LAUNCH();
  return 0;
}

size_t kdn_diag_gain_workspace_size(int B, int T, int H, int K) {
  const int64_t NT = cdiv(T, kVecChunk);  // covers both chunkings (kVecChunk <= kGainChunk)
  // maps (4) + carry (1) per (b, h, chunk, channel), [B,H,K] precision partials, then the two-level
  // carry's group composites (4) and group start values (1)
  return (size_t)((int64_t)B * H * NT * K * 5 + (int64_t)B * H * K +
                  (int64_t)B * H * cdiv(NT, kCarryGroup) * K * 5) * sizeof(float);
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
  if (gain_vec_ok(K) && aligned16(k) && aligned16(alpha) && aligned16(omega) && aligned16(kappa) &&
      aligned16(p_prev) && (prec_mode == 0 || aligned16(initial_precision))) {
    const int NV = cdiv(T, kVecChunk), tiles = B * H * NV, tpb = 256 / (K / kCPT);
    float* carry_v = maps + (int64_t)B * H * NV * K * 4;
    hipLaunchKernelGGL(diag_gain_map_v_kernel, dim3(cdiv(tiles, tpb)), dim3(256), 0, stream, k, alpha, omega, r, B, T,
                       H, K, NV, info_scale, maps);
    if (NV > 2 * kCarryGroup) {  // two-level carry
      const int NG = cdiv(NV, kCarryGroup);
      float* grp = maps + (int64_t)B * H * NV * K * 5 + (int64_t)B * H * K;
      float4* gmaps = reinterpret_cast<float4*>(grp);
      hipLaunchKernelGGL(diag_gain_group_map_kernel, dim3(B * H, NG), dim3(bs), 0, stream, (const float4*)maps, K, NV,
                         NG, gmaps);
      hipLaunchKernelGGL(diag_gain_group_fill_kernel, dim3(B * H, NG), dim3(bs), 0, stream, (const float4*)maps,
                         (const float4*)gmaps, initial_precision, prec_mode, H, K, NV, NG, carry_v, final_precision);
    } else {
      hipLaunchKernelGGL(diag_gain_carry_v_kernel, dim3(B * H), dim3(bs), 0, stream, (const float4*)maps,
                         initial_precision, prec_mode, H, K, NV, carry_v, final_precision);
    }
    hipLaunchKernelGGL(diag_gain_emit_v_kernel, dim3(cdiv(tiles, tpb)), dim3(256), 0, stream, k, alpha, omega, r,
                       carry_v, B, T, H, K, NV, info_scale, kappa, p_prev, D);
    KDN_CHECK_LAUNCH();
    return 0;
  }
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
  float* dpart_out = d_initial_precision ? (prec_mode == 1 ? d_initial_precision : dpart) : nullptr;
  if (gain_vec_ok(K) && aligned16(k) && aligned16(alpha) && aligned16(omega) && aligned16(dkappa) &&
      aligned16(p_prev) && aligned16(omega_raw) && aligned16(dk) && aligned16(dalpha) && aligned16(domega_raw) &&
      (prec_mode == 0 || (aligned16(initial_precision) && aligned16(dpart_out)))) {
    const int NV = cdiv(T, kVecChunk), tiles = B * H * NV, tpb = 256 / (K / kCPT);
    float* carry_v = ab + (int64_t)B * H * NV * K * 4;
    float* dpart_v = carry_v + (int64_t)B * H * NV * K;
    float* dpart_out_v = d_initial_precision ? (prec_mode == 1 ? d_initial_precision : dpart_v) : nullptr;
    dpart = dpart_v;
    hipLaunchKernelGGL(diag_gain_bwd_map_v_kernel, dim3(cdiv(tiles, tpb)), dim3(256), 0, stream, k, alpha, omega, r,
                       dkappa, p_prev, D, B, T, H, K, NV, info_scale, ab, G_scratch);
    if (NV > 2 * kCarryGroup) {  // two-level carry
      const int NG = cdiv(NV, kCarryGroup);
      float* grp = ab + (int64_t)B * H * NV * K * 5 + (int64_t)B * H * K;
      float2* gab = reinterpret_cast<float2*>(grp);
      hipLaunchKernelGGL(diag_gain_bwd_group_map_kernel, dim3(B * H, NG), dim3(bs), 0, stream, (const float2*)ab, K,
                         NV, NG, gab);
      hipLaunchKernelGGL(diag_gain_bwd_group_fill_kernel, dim3(B * H, NG), dim3(bs), 0, stream, (const float2*)ab,
                         (const float2*)gab, d_final_precision, final_precision, K, NV, NG, carry_v);
    } else {
      hipLaunchKernelGGL(diag_gain_bwd_carry_v_kernel, dim3(B * H), dim3(bs), 0, stream, (const float2*)ab,
                         d_final_precision, final_precision, H, K, NV, carry_v);
    }
    hipLaunchKernelGGL(diag_gain_bwd_emit_v_kernel, dim3(cdiv(tiles, tpb)), dim3(256), 0, stream, k, alpha, omega, r,
                       dkappa, p_prev, D, G_scratch, carry_v, omega_raw, r_raw, initial_precision, prec_mode, B, T, H,
                       K, NV, info_scale, dk, dalpha, domega_raw, dr_raw, dpart_out_v);
  } else {
    hipLaunchKernelGGL(diag_gain_bwd_map_kernel, dim3(NT, B * H), dim3(bs), 0, stream, k, alpha, omega, r, dkappa,
                       p_prev, D, T, H, K, NT, info_scale, ab, G_scratch);
    hipLaunchKernelGGL(diag_gain_bwd_carry_kernel, dim3(B * H), dim3(bs), 0, stream, ab, d_final_precision,
                       final_precision, H, K, NT, carry);
    hipLaunchKernelGGL(diag_gain_bwd_emit_kernel, dim3(NT, B * H), dim3(bs), 0, stream, k, alpha, omega, r, dkappa,
                       p_prev, D, G_scratch, carry, omega_raw, r_raw, initial_precision, prec_mode, T, H, K, NT,
                       info_scale, dk, dalpha, domega_raw, dr_raw, dpart_out);
  }
  if (d_initial_precision && prec_mode == 0)
    hipLaunchKernelGGL(sum_over_batch_kernel, dim3(cdiv(H, 256)), dim3(256), 0, stream, dpart, B, H,
                       d_initial_precision);
  KDN_CHECK_LAUNCH();
  return 0;
}

}  // extern "C"

// ---------------------------------------------------------------- fused diag frontend + gain
namespace {
struct FrontLayout {  // float offsets into the workspace (each 64-float aligned)
  int64_t maps, tsum, carry, grp, ab, lcarry, tdg, G, D, partA, partdt, dpart, seg, segA, total;
};
inline int64_t al64(int64_t x) { return (x + 63) / 64 * 64; }
constexpr int kFrontReduceSegments = 32;
constexpr int64_t kFrontMaxElems = int64_t(1) << 30;  // per launch, so 32-bit byte offsets of f32 arrays hold
// Batch rows per launch of the tile kernels.
inline int front_batch_chunk(int B, int T, int H, int K) {
  const int64_t per_b = (int64_t)T * H * K;
  return (int)std::max<int64_t>(1, std::min<int64_t>(B, kFrontMaxElems / per_b));
}
// The args of batch rows [b0, b0 + Bc).
template <typename TX>
FrontArgs<TX> front_shift(const FrontArgs<TX>& a, int b0, int Bc) {
  FrontArgs<TX> c = a;
  const int64_t e = (int64_t)b0 * a.T * a.H * a.K, r = (int64_t)b0 * a.T * a.H;
  c.k = a.k + e, c.f = a.f + e, c.z = a.z + e, c.knorm = a.knorm + r, c.y = a.y + r, c.B = Bc;
  return c;
}
FrontLayout front_layout(int B, int T, int H, int K) {
  const int64_t NV = cdiv(T, kVecChunk), NG = cdiv(NV, kCarryGroup), BHK = (int64_t)B * H * K;
  FrontLayout L{};
  int64_t o = 0;
  L.maps = o; o += al64(BHK * NV * 4);   // forward tile maps; the backward's (A, B) maps reuse it
  L.ab = L.maps;
  L.tsum = o; o += al64(BHK * NV);       // forward tile log-decay sums; backward tile dG sums reuse it
  L.tdg = L.tsum;
  L.carry = o; o += al64(BHK * NV);      // forward tile carries; backward lambda carries
  L.lcarry = L.carry;
  L.grp = o; o += al64(BHK * NG * 5);    // two-level carry composites and start values
  L.G = o; o += al64((int64_t)B * T * H);
  L.D = o; o += al64((int64_t)B * T * H);
  L.partA = o; o += al64((int64_t)B * NV * H);
  L.partdt = o; o += al64(BHK * NV);
  L.dpart = o; o += al64((int64_t)B * H);
  L.seg = o; o += al64((int64_t)kFrontReduceSegments * H * K);
  L.segA = o; o += al64((int64_t)kFrontReduceSegments * H);
  L.total = o;
  return L;
}
bool front_args_ok(const void* k_raw, const float* k_norm, const uint16_t* f, const uint16_t* z, const uint16_t* y,
                   const float* A_log, const float* dt_bias, const float* mu_param, const float* prec0,
                   int prec_mode, int B, int T, int H, int K, int chunk) {
  if (B <= 0 || T <= 0 || H <= 0 || (K != 64 && K != 128) || chunk <= 0 || chunk % kVecChunk != 0) return false;
  if (!k_raw || !k_norm || !f || !z || !y || !A_log || !dt_bias) return false;
  if ((int64_t)T * H * K > kFrontMaxElems) return false;  // one batch row must fit the 32-bit offsets
  if (prec_mode != 0 && prec_mode != 1) return false;
  if (mu_param ? (prec0 != nullptr || prec_mode != 0) : prec0 == nullptr) return false;
  return aligned16(k_raw) && aligned16(f) && aligned16(z) && aligned16(dt_bias) &&
         (prec_mode == 0 || aligned16(prec0));
}
template <typename TX>
FrontArgs<TX> front_args(const void* k_raw, const float* k_norm, const uint16_t* f, const uint16_t* z,
                         const uint16_t* y, const float* A_log, const float* dt_bias, int B, int T, int H, int K,
                         int chunk, float info_scale) {
  return FrontArgs<TX>{(const TX*)k_raw, k_norm, f, z, y, A_log, dt_bias, B, T, H, K, cdiv(T, kVecChunk),
                       chunk / kVecChunk, info_scale};
}

template <typename TX>
int front_fwd(const FrontArgs<TX>& a, const float* mu_param, const float* prec0, int prec_mode, float* g_cumsum,
              float* kappa, float* final_precision, float* saved, float* ws, hipStream_t stream) {
  const FrontLayout L = front_layout(a.B, a.T, a.H, a.K);
  const int NV = a.NV, tpb = 256 / (a.K / kCPT), bs = gain_block(a.K);
  float* maps = ws + L.maps;
  float* tsum = ws + L.tsum;
  float* carry = ws + L.carry;  // the tiles' entry precisions (saved: every even token's, for the backward)
  if (mu_param) prec0 = mu_param, prec_mode = 2;  // the kernels form mu = 0.1 + softplus(mu_param)
  const int Bc = front_batch_chunk(a.B, a.T, a.H, a.K);
  const int64_t ev = (int64_t)a.H * NV * a.K, ee = (int64_t)a.T * a.H * a.K;  // per batch row
  for (int b0 = 0; b0 < a.B; b0 += Bc) {
    const int nb = std::min(Bc, a.B - b0);
    hipLaunchKernelGGL((diag_front_map_kernel<TX>), dim3(cdiv((int64_t)nb * a.H * NV, tpb)), dim3(256), 0, stream,
                       front_shift(a, b0, nb), maps + b0 * ev * 4, tsum + b0 * ev);
  }
  if (NV > 2 * kCarryGroup) {  // two-level carry
    const int NG = cdiv(NV, kCarryGroup);
    float4* gmaps = reinterpret_cast<float4*>(ws + L.grp);
    hipLaunchKernelGGL(diag_gain_group_map_kernel, dim3(a.B * a.H, NG), dim3(bs), 0, stream, (const float4*)maps, a.K,
                       NV, NG, gmaps);
    hipLaunchKernelGGL(diag_gain_group_fill_kernel, dim3(a.B * a.H, NG), dim3(bs), 0, stream, (const float4*)maps,
                       (const float4*)gmaps, prec0, prec_mode, a.H, a.K, NV, NG, carry, final_precision);
  } else {
    hipLaunchKernelGGL(diag_gain_carry_v_kernel, dim3(a.B * a.H), dim3(bs), 0, stream, (const float4*)maps, prec0,
                       prec_mode, a.H, a.K, NV, carry, final_precision);
  }
  for (int b0 = 0; b0 < a.B; b0 += Bc) {
    const int nb = std::min(Bc, a.B - b0);
    hipLaunchKernelGGL((diag_front_emit_kernel<TX>), dim3(cdiv((int64_t)nb * a.H * NV, tpb)), dim3(256), 0, stream,
                       front_shift(a, b0, nb), carry + b0 * ev, tsum + b0 * ev, g_cumsum + b0 * ee, kappa + b0 * ee,
                       saved ? saved + b0 * ev * kPairs : nullptr);
  }
  KDN_CHECK_LAUNCH();
  return 0;
}

template <typename TX>
int front_bwd(const FrontArgs<TX>& a, const float* mu_param, const float* prec0, int prec_mode, const float* saved,
              const float* final_precision, const float* d_g_cumsum, const float* d_kappa, const uint16_t* d_k_memory,
              const float* d_final_precision, void* dk_raw, uint16_t* d_ret, uint16_t* d_omega, uint16_t* d_r,
              float* dA_log, float* ddt_bias, float* d_mu_param, float* d_prec, float* ws, hipStream_t stream) {
  const FrontLayout L = front_layout(a.B, a.T, a.H, a.K);
  const int NV = a.NV, tpb = 256 / (a.K / kCPT), bs = gain_block(a.K);
  float* ab = ws + L.ab;
  float* lcarry = ws + L.lcarry;
  float* tdg = ws + L.tdg;
  float* G = ws + L.G;
  float* D = ws + L.D;
  if (mu_param) prec0 = mu_param, prec_mode = 2;  // the kernels form mu = 0.1 + softplus(mu_param)
  const int Bc = front_batch_chunk(a.B, a.T, a.H, a.K);
  const int64_t ev = (int64_t)a.H * NV * a.K, ee = (int64_t)a.T * a.H * a.K, er = (int64_t)a.T * a.H;
  for (int b0 = 0; b0 < a.B; b0 += Bc) {
    const int nb = std::min(Bc, a.B - b0);
    hipLaunchKernelGGL((diag_front_bwd_map_kernel<TX>), dim3(cdiv((int64_t)nb * a.H * NV, tpb)), dim3(256), 0, stream,
                       front_shift(a, b0, nb), saved + b0 * ev * kPairs, d_kappa + b0 * ee, d_g_cumsum + b0 * ee,
                       ab + b0 * ev * 2, tdg + b0 * ev, G + b0 * er, D + b0 * er);
  }
  if (NV > 2 * kCarryGroup) {  // two-level carry
    const int NG = cdiv(NV, kCarryGroup);
    float2* gab = reinterpret_cast<float2*>(ws + L.grp);
    hipLaunchKernelGGL(diag_gain_bwd_group_map_kernel, dim3(a.B * a.H, NG), dim3(bs), 0, stream, (const float2*)ab,
                       a.K, NV, NG, gab);
    hipLaunchKernelGGL(diag_gain_bwd_group_fill_kernel, dim3(a.B * a.H, NG), dim3(bs), 0, stream, (const float2*)ab,
                       (const float2*)gab, d_final_precision, final_precision, a.K, NV, NG, lcarry);
  } else {
    hipLaunchKernelGGL(diag_gain_bwd_carry_v_kernel, dim3(a.B * a.H), dim3(bs), 0, stream, (const float2*)ab,
                       d_final_precision, final_precision, a.H, a.K, NV, lcarry);
  }
  const bool want_prec = d_mu_param || d_prec;
  float* dprec_out = want_prec ? (prec_mode == 1 ? d_prec : ws + L.dpart) : nullptr;  // [B,H,K] or [B,H]
  for (int b0 = 0; b0 < a.B; b0 += Bc) {
    const int nb = std::min(Bc, a.B - b0);
    const int64_t ep = prec_mode == 1 ? (int64_t)a.H * a.K : a.H;  // per batch row of [B,H,K] / [B,H]
    hipLaunchKernelGGL((diag_front_bwd_emit_kernel<TX>), dim3(cdiv((int64_t)nb * a.H * NV, tpb)), dim3(256), 0, stream,
                       front_shift(a, b0, nb), saved + b0 * ev * kPairs, lcarry + b0 * ev, d_kappa + b0 * ee,
                       d_g_cumsum + b0 * ee, tdg + b0 * ev, G + b0 * er, D + b0 * er,
                       d_k_memory ? (const bf16_t*)d_k_memory + b0 * ee : nullptr,
                       prec_mode == 1 ? prec0 + b0 * ep : prec0, prec_mode,
                       dk_raw ? (TX*)dk_raw + b0 * ee : nullptr, (bf16_t*)d_ret + b0 * ee, (bf16_t*)d_omega + b0 * ee,
                       (bf16_t*)d_r + b0 * er, dA_log ? ws + L.partA + (int64_t)b0 * NV * a.H : nullptr,
                       ddt_bias ? ws + L.partdt + b0 * ev : nullptr, dprec_out ? dprec_out + b0 * ep : nullptr);
  }
  // dA_log [H] and d dt_bias [H K] from the B*NV partial rows, in row segments (S launches' worth of
  // workgroups) and then the segment sums, and the prior's VJP (sum over b of the per-row cotangents) with
  // the second: two launches
  const int NP = a.B * NV, HK = a.H * a.K;
  const int S = std::max(1, std::min(kFrontReduceSegments, NP / 64));
  PartSegs fin{};
  auto add = [](PartSegs& P, const float* part, int n, float* out) { P.seg[P.nseg++] = PartSeg{part, n, n, out}; };
  if (S > 1) {
    PartSegs rows{};
    if (dA_log) add(rows, ws + L.partA, a.H, ws + L.segA);
    if (ddt_bias) add(rows, ws + L.partdt, HK, ws + L.seg);
    if (rows.nseg > 0)
      hipLaunchKernelGGL(reduce_partials_multi_kernel, dim3(part_segs_blocks(rows), S), dim3(256), 0, stream, rows,
                         NP);
    if (dA_log) add(fin, ws + L.segA, a.H, dA_log);
    if (ddt_bias) add(fin, ws + L.seg, HK, ddt_bias);
  } else {
    if (dA_log) add(fin, ws + L.partA, a.H, dA_log);
    if (ddt_bias) add(fin, ws + L.partdt, HK, ddt_bias);
  }
  if (want_prec && prec_mode != 1) {  // d mu_param = sigmoid(mu_param) sum_b part (or the [H] prior's sum)
    fin.mu_param = mu_param;
    fin.dmu_rows = ws + L.dpart;
    fin.nrows = a.B;
    fin.rows_to_param = 1;
    fin.H = a.H;
    if (d_mu_param) fin.dmu_param = d_mu_param;
    else fin.dmu_sum = d_prec;
  }
  const int nfin = part_segs_blocks(fin);
  if (nfin > 0)
    hipLaunchKernelGGL(reduce_partials_multi_kernel, dim3(nfin), dim3(256), 0, stream, fin, S > 1 ? S : NP);
  KDN_CHECK_LAUNCH();
  return 0;
}
}  // namespace

extern "C" {

size_t kdn_diag_front_saved_size(int B, int T, int H, int K) {
  if (B <= 0 || T <= 0 || H <= 0 || K <= 0) return 0;
  return (size_t)((int64_t)B * H * cdiv(T, kVecChunk) * kPairs * K) * sizeof(float);
}

size_t kdn_diag_front_workspace_size(int B, int T, int H, int K) {
  if (B <= 0 || T <= 0 || H <= 0 || K <= 0) return 0;
  return (size_t)front_layout(B, T, H, K).total * sizeof(float);
}

int kdn_diag_front_fwd(const void* k_raw, int k_bf16, const float* k_norm, const uint16_t* retention_raw,
                       const uint16_t* omega_raw, const uint16_t* r_raw, const float* A_log, const float* dt_bias,
                       const float* mu_param, const float* initial_precision, int prec_mode, int B, int T, int H,
                       int K, int chunk, float info_scale, float* g_cumsum, float* kappa, float* final_precision,
                       float* saved, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!front_args_ok(k_raw, k_norm, retention_raw, omega_raw, r_raw, A_log, dt_bias, mu_param, initial_precision,
                     prec_mode, B, T, H, K, chunk))
    return KDN_ERR_ARG;
  if (!g_cumsum || !kappa || !aligned16(g_cumsum) || !aligned16(kappa) || !aligned16(saved) ||
      !aligned16(workspace) || !(info_scale > 0.f))
    return KDN_ERR_ARG;
  if (workspace_bytes < kdn_diag_front_workspace_size(B, T, H, K)) return KDN_ERR_ARG;
  float* ws = (float*)workspace;
  if (k_bf16)
    return front_fwd(front_args<bf16_t>(k_raw, k_norm, retention_raw, omega_raw, r_raw, A_log, dt_bias, B, T, H, K,
                                        chunk, info_scale),
                     mu_param, initial_precision, prec_mode, g_cumsum, kappa, final_precision, saved, ws, stream);
  return front_fwd(front_args<float>(k_raw, k_norm, retention_raw, omega_raw, r_raw, A_log, dt_bias, B, T, H, K, chunk,
                                     info_scale),
                   mu_param, initial_precision, prec_mode, g_cumsum, kappa, final_precision, saved, ws, stream);
}

int kdn_diag_front_bwd(const void* k_raw, int k_bf16, const float* k_norm, const uint16_t* retention_raw,
                       const uint16_t* omega_raw, const uint16_t* r_raw, const float* A_log, const float* dt_bias,
                       const float* mu_param, const float* initial_precision, int prec_mode, const float* saved,
                       const float* final_precision, const float* d_g_cumsum, const float* d_kappa,
                       const uint16_t* d_k_memory, const float* d_final_precision, int B, int T, int H, int K,
                       int chunk, float info_scale, void* dk_raw, uint16_t* d_retention_raw, uint16_t* d_omega_raw,
                       uint16_t* d_r_raw, float* dA_log, float* ddt_bias, float* d_mu_param,
                       float* d_initial_precision, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!front_args_ok(k_raw, k_norm, retention_raw, omega_raw, r_raw, A_log, dt_bias, mu_param, initial_precision,
                     prec_mode, B, T, H, K, chunk))
    return KDN_ERR_ARG;
  if (!saved || !d_g_cumsum || !d_kappa || !d_retention_raw || !d_omega_raw || !d_r_raw) return KDN_ERR_ARG;
  if (d_final_precision && !final_precision) return KDN_ERR_ARG;
  if (d_mu_param && !mu_param) return KDN_ERR_ARG;
  if (d_initial_precision && mu_param) return KDN_ERR_ARG;
  if (!aligned16(saved) || !aligned16(d_g_cumsum) || !aligned16(d_kappa) || !aligned16(d_k_memory) ||
      !aligned16(dk_raw) || !aligned16(d_retention_raw) || !aligned16(d_omega_raw) || !aligned16(ddt_bias) ||
      !aligned16(workspace) || (prec_mode == 1 && !aligned16(d_initial_precision)) || !(info_scale > 0.f))
    return KDN_ERR_ARG;
  if (workspace_bytes < kdn_diag_front_workspace_size(B, T, H, K)) return KDN_ERR_ARG;
  float* ws = (float*)workspace;
  if (k_bf16)
    return front_bwd(front_args<bf16_t>(k_raw, k_norm, retention_raw, omega_raw, r_raw, A_log, dt_bias, B, T, H, K,
                                        chunk, info_scale),
                     mu_param, initial_precision, prec_mode, saved, final_precision, d_g_cumsum, d_kappa, d_k_memory,
                     d_final_precision, dk_raw, d_retention_raw, d_omega_raw, d_r_raw, dA_log, ddt_bias, d_mu_param,
                     d_initial_precision, ws, stream);
  return front_bwd(front_args<float>(k_raw, k_norm, retention_raw, omega_raw, r_raw, A_log, dt_bias, B, T, H, K, chunk,
                                     info_scale),
                   mu_param, initial_precision, prec_mode, saved, final_precision, d_g_cumsum, d_kappa, d_k_memory,
                   d_final_precision, dk_raw, d_retention_raw, d_omega_raw, d_r_raw, dA_log, ddt_bias, d_mu_param,
                   d_initial_precision, ws, stream);
}

}  // extern "C"
