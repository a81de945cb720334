// Single-token step of the KDN memory recurrence (decode with a carried state).
//
// The reference runs only fixed-length sequences and has no step kernel; its recurrence is the
// tokenwise one of iso_kdn_naive.py:308-332 and diag_kdn_naive.py:479-500:
//   S_hat = diag(e) S,  e = 2^g (g = the token's base-2 log decay, the chunked scan's g_cumsum
//   at T = 1);  delta = v - S_hat^T k;  S = S_hat + kappa delta^T;  o = scale S^T q.
// For the isotropic variant kappa = beta k_hat and q, k are L2-normalised here exactly as the
// chunked scan normalises them (x * rsqrt(sum x^2 + 1e-6)); the diagonal variant takes
// normalised q, k and an explicit kappa.  State layout is the scan's h0 / ht layout
// [B,H,K,V] fp32, so a chunked prefill's final state feeds this kernel directly.
//
// One workgroup per (b, h, 32-column slice of V), 256 threads: thread t owns columns
// 4 (t & 7) .. +3 of the slice and rows rg + 32 j (rg = t >> 3, j < K / 32), so each row's 128
// bytes of the slice are read and written by 8 neighbouring lanes (float4 each).  The two sums
// over K (delta and o) reduce over lane bits 3..5 with xor shuffles, then over the 4 waves in LDS.
// HBM traffic per token is 2 K V 4 bytes of state (read + write) plus the vectors.
#include "kdn_common.h"

namespace {

constexpr float kL2Eps = 1e-6f;

__device__ __forceinline__ float4 f4_fma(float a, const float4& x, const float4& y) {
  return float4{fmaf(a, x.x, y.x), fmaf(a, x.y, y.y), fmaf(a, x.z, y.z), fmaf(a, x.w, y.w)};
}
__device__ __forceinline__ float4 f4_scale(float a, const float4& x) { return float4{a * x.x, a * x.y, a * x.z, a * x.w}; }
__device__ __forceinline__ float4 f4_add(const float4& x, const float4& y) {
  return float4{x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w};
}
__device__ __forceinline__ float4 f4_sub(const float4& x, const float4& y) {
  return float4{x.x - y.x, x.y - y.y, x.z - y.z, x.w - y.w};
}
__device__ __forceinline__ float4 f4_xor(const float4& x, int m) {
  return float4{__shfl_xor(x.x, m, 64), __shfl_xor(x.y, m, 64), __shfl_xor(x.z, m, 64), __shfl_xor(x.w, m, 64)};
}

// Sum of x over the 32 row groups of the workgroup for this thread's 4 columns; valid in every
// thread.  `red` is [4 waves][8 column groups] of float4; the caller separates two uses by a
// barrier or uses two buffers.
__device__ __forceinline__ float4 rows_sum(float4 x, float4* red) {
  x = f4_add(x, f4_xor(x, 8));
  x = f4_add(x, f4_xor(x, 16));
  x = f4_add(x, f4_xor(x, 32));
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane < 8) red[w * 8 + lane] = x;
  __syncthreads();
  const int c = lane & 7;
  return f4_add(f4_add(red[c], red[8 + c]), f4_add(red[16 + c], red[24 + c]));
}

template <typename T> __device__ __forceinline__ float4 ld4(const T* p);
template <> __device__ __forceinline__ float4 ld4<float>(const float* p) { return *reinterpret_cast<const float4*>(p); }
template <> __device__ __forceinline__ float4 ld4<bf16_t>(const bf16_t* p) {
  const uint2 u = *reinterpret_cast<const uint2*>(p);
  return float4{__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                __uint_as_float(u.y & 0xffff0000u)};
}
template <typename T> __device__ __forceinline__ void st4(T* p, const float4& x);
template <> __device__ __forceinline__ void st4<float>(float* p, const float4& x) { *reinterpret_cast<float4*>(p) = x; }
template <> __device__ __forceinline__ void st4<bf16_t>(bf16_t* p, const float4& x) {
  const uint2 u{(uint32_t)f2bf(x.x) | ((uint32_t)f2bf(x.y) << 16), (uint32_t)f2bf(x.z) | ((uint32_t)f2bf(x.w) << 16)};
  *reinterpret_cast<uint2*>(p) = u;
}

// grid (B * H * V / 32), block 256.
template <int K, int V, typename TI, typename TO, bool ISO>
__global__ __launch_bounds__(256) void mem_step_kernel(const TI* __restrict__ q, const TI* __restrict__ k,
                                                       const float* __restrict__ kappa_or_beta,
                                                       const TI* __restrict__ v, const float* __restrict__ g,
                                                       float scale, float* __restrict__ state, TO* __restrict__ o) {
  constexpr int NS = V / 32, R = K / 32;
  __shared__ float4 red[2][32];
  const int64_t bh = blockIdx.x / NS;
  const int slice = blockIdx.x % NS, t = threadIdx.x, lane = t & 63, c4 = t & 7, rg = t >> 3;
  const TI* qp = q + bh * K;
  const TI* kp = k + bh * K;
  float qs = 1.f, ks = 1.f;
  if (ISO) {  // every wave forms both norms itself (K <= 128: two elements per lane)
    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int i = lane; i < K; i += 64) {
      const float a = ld(qp, i), b = ld(kp, i);
      sq = fmaf(a, a, sq);
      sk = fmaf(b, b, sk);
    }
    qs = 1.f / sqrtf(wave_sum(sq) + kL2Eps);
    ks = 1.f / sqrtf(wave_sum(sk) + kL2Eps);
  }
  const float beta = ISO ? kappa_or_beta[bh] : 0.f;
  const int col = slice * 32 + 4 * c4;
  float* sp = state + bh * K * V + col;
  float4 S[R];
  float kr[R], qr[R], kap[R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int row = rg + 32 * j;
    S[j] = *reinterpret_cast<const float4*>(sp + (int64_t)row * V);
    kr[j] = ld(kp, row) * ks;
    qr[j] = ld(qp, row) * qs;
    kap[j] = ISO ? beta * kr[j] : kappa_or_beta[bh * K + row];
    S[j] = f4_scale(exp2f(g[bh * K + row]), S[j]);
  }
  float4 acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < R; ++j) acc = f4_fma(kr[j], S[j], acc);
  const float4 delta = f4_sub(ld4(v + bh * V + col), rows_sum(acc, red[0]));
  acc = float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < R; ++j) {
    S[j] = f4_fma(kap[j], delta, S[j]);
    *reinterpret_cast<float4*>(sp + (int64_t)(rg + 32 * j) * V) = S[j];
    acc = f4_fma(qr[j], S[j], acc);
  }
  const float4 out = rows_sum(acc, red[1]);
  if (t < 8) st4(o + bh * V + col, f4_scale(scale, out));
}

// Sum of x over the 32 row groups (one value per row group, the same in its 8 column lanes);
// valid in every thread.  `red` holds 4 floats.
__device__ __forceinline__ float rows_sum_scalar(float x, float* red) {
  x += __shfl_xor(x, 8, 64);
  x += __shfl_xor(x, 16, 64);
  x += __shfl_xor(x, 32, 64);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) red[w] = x;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

// One token of the full Kalman step: the gain from the carried precision, then the memory
// update of mem_step_kernel.  grid (B * H * V / 32), block 256.
//   iso:  p = 1 / c;  z = a p + w;  beta = z / (r + z);  p' = r z / (r + s z)  (unit keys; s = info_scale / K)
//   diag: p = 1 / c;  p_hat = alpha^2 p + w;  kappa = p_hat k / (r + sum_i p_hat_i k_i^2);
//         p' = p_hat / (1 + s k^2 p_hat / r)                                   (s = info_scale)
// c' = 1 / p' goes to prec_out (written by the workgroup of the first column slice; every
// workgroup of a (b, h) reads prec_in, so the two must not alias).
template <int K, int V, typename TI, typename TO, bool ISO>
__global__ __launch_bounds__(256) void kalman_step_kernel(
    const TI* __restrict__ q, const TI* __restrict__ k, const TI* __restrict__ v, const float* __restrict__ g,
    const float* __restrict__ ga, const float* __restrict__ gw, const float* __restrict__ gr,
    const float* __restrict__ kg, const float* __restrict__ prec_in, float* __restrict__ prec_out, float scale,
    float s, float* __restrict__ state, TO* __restrict__ o) {
  constexpr int NS = V / 32, R = K / 32;
  __shared__ float4 red[2][32];
  __shared__ float redg[4];
  const int64_t bh = blockIdx.x / NS;
  const int slice = blockIdx.x % NS, t = threadIdx.x, lane = t & 63, c4 = t & 7, rg = t >> 3;
  const TI* qp = q + bh * K;
  const TI* kp = k + bh * K;
  float qs = 1.f, ks = 1.f;
  if (ISO) {
    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int i = lane; i < K; i += 64) {
      const float a = ld(qp, i), b = ld(kp, i);
      sq = fmaf(a, a, sq);
      sk = fmaf(b, b, sk);
    }
    qs = 1.f / sqrtf(wave_sum(sq) + kL2Eps);
    ks = 1.f / sqrtf(wave_sum(sk) + kL2Eps);
  }
  const float rt = gr[bh], ir = 1.f / rt;
  const int col = slice * 32 + 4 * c4;
  float* sp = state + bh * K * V + col;
  float4 S[R];
  float kr[R], qr[R], kap[R];
  float beta = 0.f;
  if (ISO) {
    const float p = 1.f / prec_in[bh];
    const float z = ga[bh] * p + gw[bh];
    beta = z / (rt + z);
    if (slice == 0 && t == 0) prec_out[bh] = (rt + s * z) / (rt * z);
  }
  float ph[R], kgv[R], part = 0.f;
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int row = rg + 32 * j;
    S[j] = *reinterpret_cast<const float4*>(sp + (int64_t)row * V);
    kr[j] = ld(kp, row) * ks;
    qr[j] = ld(qp, row) * qs;
    if (!ISO) {
      const int64_t e = bh * K + row;
      const float al = ga[e];
      kgv[j] = kg ? kg[e] : kr[j];
      ph[j] = al * al / prec_in[e] + gw[e];
      part = fmaf(ph[j] * kgv[j], kgv[j], part);
    }
    S[j] = f4_scale(exp2f(g[bh * K + row]), S[j]);
  }
  if (!ISO) {
    const float iD = 1.f / (rt + rows_sum_scalar(part, redg));
#pragma unroll
    for (int j = 0; j < R; ++j) {
      kap[j] = ph[j] * kgv[j] * iD;
      if (slice == 0 && c4 == 0) prec_out[bh * K + rg + 32 * j] = (1.f + s * kgv[j] * kgv[j] * ir * ph[j]) / ph[j];
    }
  } else {
#pragma unroll
    for (int j = 0; j < R; ++j) kap[j] = beta * kr[j];
  }
  float4 acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < R; ++j) acc = f4_fma(kr[j], S[j], acc);
  const float4 delta = f4_sub(ld4(v + bh * V + col), rows_sum(acc, red[0]));
  acc = float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < R; ++j) {
    S[j] = f4_fma(kap[j], delta, S[j]);
    *reinterpret_cast<float4*>(sp + (int64_t)(rg + 32 * j) * V) = S[j];
    acc = f4_fma(qr[j], S[j], acc);
  }
  const float4 out = rows_sum(acc, red[1]);
  if (t < 8) st4(o + bh * V + col, f4_scale(scale, out));
}

template <int K, int V, typename TI, typename TO>
void launch_kalman(bool iso, const void* q, const void* k, const void* v, const float* g, const float* ga,
                   const float* gw, const float* gr, const float* kg, const float* pin, float* pout, int BH,
                   float scale, float s, float* state, void* o, hipStream_t stream) {
  const dim3 grid(BH * (V / 32)), block(256);
  if (iso)
    hipLaunchKernelGGL((kalman_step_kernel<K, V, TI, TO, true>), grid, block, 0, stream, (const TI*)q, (const TI*)k,
                       (const TI*)v, g, ga, gw, gr, kg, pin, pout, scale, s, state, (TO*)o);
  else
    hipLaunchKernelGGL((kalman_step_kernel<K, V, TI, TO, false>), grid, block, 0, stream, (const TI*)q, (const TI*)k,
                       (const TI*)v, g, ga, gw, gr, kg, pin, pout, scale, s, state, (TO*)o);
}

template <int K, int V>
void launch_kalman_kv(bool iso, const void* q, const void* k, const void* v, int qkv_bf16, const float* g,
                      const float* ga, const float* gw, const float* gr, const float* kg, const float* pin, float* pout,
                      int BH, float scale, float s, float* state, void* o, int o_bf16, hipStream_t stream) {
  if (qkv_bf16 && o_bf16)
    launch_kalman<K, V, bf16_t, bf16_t>(iso, q, k, v, g, ga, gw, gr, kg, pin, pout, BH, scale, s, state, o, stream);
  else if (qkv_bf16)
    launch_kalman<K, V, bf16_t, float>(iso, q, k, v, g, ga, gw, gr, kg, pin, pout, BH, scale, s, state, o, stream);
  else if (o_bf16)
    launch_kalman<K, V, float, bf16_t>(iso, q, k, v, g, ga, gw, gr, kg, pin, pout, BH, scale, s, state, o, stream);
  else
    launch_kalman<K, V, float, float>(iso, q, k, v, g, ga, gw, gr, kg, pin, pout, BH, scale, s, state, o, stream);
}

template <int K, int V, typename TI, typename TO>
void launch_step(bool iso, const void* q, const void* k, const float* kb, const void* v, const float* g, int BH,
                 float scale, float* state, void* o, hipStream_t stream) {
  const dim3 grid(BH * (V / 32)), block(256);
  if (iso)
    hipLaunchKernelGGL((mem_step_kernel<K, V, TI, TO, true>), grid, block, 0, stream, (const TI*)q, (const TI*)k, kb,
                       (const TI*)v, g, scale, state, (TO*)o);
  else
    hipLaunchKernelGGL((mem_step_kernel<K, V, TI, TO, false>), grid, block, 0, stream, (const TI*)q, (const TI*)k, kb,
                       (const TI*)v, g, scale, state, (TO*)o);
}

template <int K, int V>
void launch_step_kv(bool iso, const void* q, const void* k, int qkv_bf16, const float* kb, const void* v,
                    const float* g, int BH, float scale, float* state, void* o, int o_bf16, hipStream_t stream) {
  if (qkv_bf16 && o_bf16) launch_step<K, V, bf16_t, bf16_t>(iso, q, k, kb, v, g, BH, scale, state, o, stream);
  else if (qkv_bf16) launch_step<K, V, bf16_t, float>(iso, q, k, kb, v, g, BH, scale, state, o, stream);
  else if (o_bf16) launch_step<K, V, float, bf16_t>(iso, q, k, kb, v, g, BH, scale, state, o, stream);
  else launch_step<K, V, float, float>(iso, q, k, kb, v, g, BH, scale, state, o, stream);
}

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace

extern "C" {

int kdn_mem_step(const void* q, const void* k, const float* kappa_or_beta, int iso, const void* v, int qkv_bf16,
                 const float* g, int B, int H, int K, int V, float scale, float* state, void* o, int o_bf16,
                 hipStream_t stream) {
  if (B < 0 || H <= 0 || (K != 64 && K != 128) || (V != 64 && V != 128)) return KDN_ERR_ARG;
  if (B == 0) return 0;
  if (!q || !k || !kappa_or_beta || !v || !g || !state || !o) return KDN_ERR_ARG;
  // float4 state rows and 4-element vector loads / stores
  if (!aligned(state, 16) || !aligned(v, qkv_bf16 ? 8 : 16) || !aligned(o, o_bf16 ? 8 : 16)) return KDN_ERR_ARG;
  const int BH = B * H;
  const bool is_iso = iso != 0;
  if (K == 64 && V == 64) launch_step_kv<64, 64>(is_iso, q, k, qkv_bf16, kappa_or_beta, v, g, BH, scale, state, o, o_bf16, stream);
  else if (K == 64) launch_step_kv<64, 128>(is_iso, q, k, qkv_bf16, kappa_or_beta, v, g, BH, scale, state, o, o_bf16, stream);
  else if (V == 64) launch_step_kv<128, 64>(is_iso, q, k, qkv_bf16, kappa_or_beta, v, g, BH, scale, state, o, o_bf16, stream);
  else launch_step_kv<128, 128>(is_iso, q, k, qkv_bf16, kappa_or_beta, v, g, BH, scale, state, o, o_bf16, stream);
  KDN_CHECK_LAUNCH();
  return 0;
}

int kdn_kalman_step(const void* q, const void* k, const void* v, int qkv_bf16, const float* g, const float* gain_a,
                    const float* omega, const float* r, const float* k_gain, const float* precision_in,
                    float* precision_out, int iso, int B, int H, int K, int V, float scale, float info_scale,
                    float* state, void* o, int o_bf16, hipStream_t stream) {
  if (B < 0 || H <= 0 || (K != 64 && K != 128) || (V != 64 && V != 128) || !(info_scale > 0.f)) return KDN_ERR_ARG;
  if (B == 0) return 0;
  if (!q || !k || !v || !g || !gain_a || !omega || !r || !precision_in || !precision_out || !state || !o)
    return KDN_ERR_ARG;
  if (precision_in == precision_out) return KDN_ERR_ARG;  // every workgroup of a (b, h) reads precision_in
  if (!aligned(state, 16) || !aligned(v, qkv_bf16 ? 8 : 16) || !aligned(o, o_bf16 ? 8 : 16)) return KDN_ERR_ARG;
  const int BH = B * H;
  const bool is_iso = iso != 0;
  const float s = is_iso ? info_scale / (float)K : info_scale;
  const float* kg = is_iso ? nullptr : k_gain;
#define KDN_KS(KK, VV)                                                                                           \
  launch_kalman_kv<KK, VV>(is_iso, q, k, v, qkv_bf16, g, gain_a, omega, r, kg, precision_in, precision_out, BH, \
                           scale, s, state, o, o_bf16, stream)
  if (K == 64 && V == 64) KDN_KS(64, 64);
  else if (K == 64) KDN_KS(64, 128);
  else if (V == 64) KDN_KS(128, 64);
  else KDN_KS(128, 128);
#undef KDN_KS
  KDN_CHECK_LAUNCH();
  return 0;
}

}  // extern "C"

// ---------------------------------------------------------------------------------------------
// Decode projections: y[m, n] = sum_k x[m, k] W[n, k] (+ bias[n]) for a few rows m (M <= 8) and a
// bf16 weight W [N, K] (an nn.Linear weight), fp32 accumulation.  With one token per sequence the
// product reads every weight element once, so it is bound by the weight stream.  One wave per
// output row, 4 rows a workgroup (N / 4 workgroups: 576 at N = 2304, so even the narrow
// projections fill the chip; 16 lanes per row gave a quarter of that and 20% slower decode steps).
// A lane reads 16 bytes of its row per 512-column step with 8 steps in flight (a wave covers 1 KiB
// contiguous per step), x through the cache, and the row's sum meets in 6 xor shuffles.
// K % 8 == 0: a lane's 8-column segment past K (the last step of a K that is not a multiple of
// 512) loads the row's last segment instead and its weights are zeroed, so no load sits under a
// branch and a lane's loads all issue together.  gated != 0 is the fused SwiGLU gate over a
// packed [w1; w2] weight (below).
// ---------------------------------------------------------------------------------------------
namespace {

constexpr int kGemvInFlight = 8;  // steps whose weight loads are issued together
constexpr int kGemvLanes = 64;    // lanes per output row

// MM = the instantiated row capacity; rows m >= M (runtime) are neither read nor written.
// GATED: W holds 2N rows [W1; W2] (and bias 2N entries); the wave of output n also reads row N + n
// and writes silu(W1 x + b1) * (W2 x + b2), the SwiGLU gate, in fp32 before the one rounding.
template <int MM, bool GATED, typename TX, typename TY>
__global__ __launch_bounds__(256) void gemv_kernel(const TX* __restrict__ x, int64_t xs, const bf16_t* __restrict__ W,
                                                   const bf16_t* __restrict__ bias, int M, int N, int K,
                                                   TY* __restrict__ y, int64_t ys) {
  constexpr int kGemvRows = 256 / kGemvLanes, kGemvStep = 8 * kGemvLanes;
  const int t = threadIdx.x, j = t % kGemvLanes;
  const int n = blockIdx.x * kGemvRows + t / kGemvLanes;
  const bool live = n < N;
  const bf16_t* wr = W + (int64_t)(live ? n : 0) * K + 8 * j;
  const bf16_t* wr2 = wr + (int64_t)N * K;  // GATED: row N + n
  float acc[MM], acc2[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) acc[m] = 0.f, acc2[m] = 0.f;
  constexpr int U = kGemvInFlight;
  for (int k0 = 0; k0 < K; k0 += kGemvStep * U) {
    uint4 wv[U], wv2[GATED ? U : 1];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = min(k0 + kGemvStep * u + 8 * j, K - 8);  // clamped into the row
      wv[u] = *reinterpret_cast<const uint4*>(wr - 8 * j + kk);
      if constexpr (GATED) wv2[u] = *reinterpret_cast<const uint4*>(wr2 - 8 * j + kk);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (k0 + kGemvStep * u >= K) break;  // uniform: no lane has columns left
      const int kk_raw = k0 + kGemvStep * u + 8 * j;
      const bool in = kk_raw < K;  // K % 8 == 0: the whole segment is inside the row
      const int kk = in ? kk_raw : K - 8;
      const uint32_t ww[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
      float wf[8], wf2[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        wf[2 * q] = in ? __uint_as_float(ww[q] << 16) : 0.f;
        wf[2 * q + 1] = in ? __uint_as_float(ww[q] & 0xffff0000u) : 0.f;
      }
      if constexpr (GATED) {
        const uint32_t w2[4] = {wv2[u].x, wv2[u].y, wv2[u].z, wv2[u].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          wf2[2 * q] = in ? __uint_as_float(w2[q] << 16) : 0.f;
          wf2[2 * q + 1] = in ? __uint_as_float(w2[q] & 0xffff0000u) : 0.f;
        }
      }
#pragma unroll
      for (int m = 0; m < MM; ++m) {
        if (m >= M) break;
        float xf[8];
        if constexpr (sizeof(TX) == 2) {
          const uint4 xv = *reinterpret_cast<const uint4*>(x + m * xs + kk);
          const uint32_t xx[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            xf[2 * q] = __uint_as_float(xx[q] << 16);
            xf[2 * q + 1] = __uint_as_float(xx[q] & 0xffff0000u);
          }
        } else {
          const float4 a = *reinterpret_cast<const float4*>(x + m * xs + kk);
          const float4 b = *reinterpret_cast<const float4*>(x + m * xs + kk + 4);
          xf[0] = a.x, xf[1] = a.y, xf[2] = a.z, xf[3] = a.w, xf[4] = b.x, xf[5] = b.y, xf[6] = b.z, xf[7] = b.w;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          acc[m] = fmaf(wf[e], xf[e], acc[m]);
          if constexpr (GATED) acc2[m] = fmaf(wf2[e], xf[e], acc2[m]);
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MM; ++m)
#pragma unroll
    for (int o = 1; o < kGemvLanes; o <<= 1) {
      acc[m] += __shfl_xor(acc[m], o, 64);
      if constexpr (GATED) acc2[m] += __shfl_xor(acc2[m], o, 64);
    }
  if (live && j == 0) {
    const float bb = bias ? bf2f(bias[n]) : 0.f;
    const float bb2 = (GATED && bias) ? bf2f(bias[N + n]) : 0.f;
#pragma unroll
    for (int m = 0; m < MM; ++m)
      if (m < M) {
        const float v = acc[m] + bb;
        // silu(v) = v / (1 + e^-v); e^-v = inf for very negative v gives -0
        st(y, m * ys + n, GATED ? v / (1.f + __expf(-v)) * (acc2[m] + bb2) : v);
      }
  }
}

template <int MM, bool GATED>
void launch_gemv_g(const void* x, int x_bf16, int64_t xs, const bf16_t* W, const bf16_t* bias, int M, int N, int K,
                   void* y, int64_t ys, hipStream_t stream) {
  constexpr int rows = 256 / kGemvLanes;
  const dim3 grid((N + rows - 1) / rows), block(256);
  if (x_bf16)
    hipLaunchKernelGGL((gemv_kernel<MM, GATED, bf16_t, bf16_t>), grid, block, 0, stream, (const bf16_t*)x, xs, W, bias,
                       M, N, K, (bf16_t*)y, ys);
  else
    hipLaunchKernelGGL((gemv_kernel<MM, GATED, float, float>), grid, block, 0, stream, (const float*)x, xs, W, bias, M,
                       N, K, (float*)y, ys);
}

template <int MM>
void launch_gemv(const void* x, int x_bf16, int64_t xs, const bf16_t* W, const bf16_t* bias, int M, int N, int K,
                 int gated, void* y, int64_t ys, hipStream_t stream) {
  if (gated) launch_gemv_g<MM, true>(x, x_bf16, xs, W, bias, M, N, K, y, ys, stream);
  else launch_gemv_g<MM, false>(x, x_bf16, xs, W, bias, M, N, K, y, ys, stream);
}

}  // namespace

extern "C" int kdn_gemv(const void* x, int x_bf16, int64_t x_row_stride, const uint16_t* W, const uint16_t* bias,
                        int M, int N, int K, int gated, void* y, int64_t y_row_stride, hipStream_t stream) {
  if (M < 0 || M > 8 || N < 0 || K <= 0 || K % 8 || !W || !x || !y) return KDN_ERR_ARG;
  if (M == 0 || N == 0) return 0;
  // 16-byte rows: W rows are K * 2 bytes (K % 8 == 0); x rows 16-byte aligned
  if (!aligned(W, 16) || !aligned(x, 16) || (x_row_stride * (x_bf16 ? 2 : 4)) % 16) return KDN_ERR_ARG;
  if (M == 1) launch_gemv<1>(x, x_bf16, x_row_stride, W, bias, M, N, K, gated, y, y_row_stride, stream);
  else if (M == 2) launch_gemv<2>(x, x_bf16, x_row_stride, W, bias, M, N, K, gated, y, y_row_stride, stream);
  else if (M <= 4) launch_gemv<4>(x, x_bf16, x_row_stride, W, bias, M, N, K, gated, y, y_row_stride, stream);
  else launch_gemv<8>(x, x_bf16, x_row_stride, W, bias, M, N, K, gated, y, y_row_stride, stream);
  KDN_CHECK_LAUNCH();
  return 0;
}
