// Layer frontends of the KDN mixers, around the scan: the depthwise causal short convolution
// with SiLU that produces q, k, v, and the sigmoid-gated RMS norm of the mixer output.
// HBM-bound elementwise / short-window work; 16-byte accesses with consecutive threads on
// consecutive channel groups of one row.
//
// Reference behaviour restated (ngocbh/kalman-delta-networks):
//   short conv    FLA causal_conv1d(x, weight, activation="silu"), fixed length, width 4, no bias,
//                 as called per tensor by lit_gpt/diag_kdn.py:75-96 and per packed q|k|v group by
//                 lit_gpt/kdn_ops/iso_kdn_chunk.py:47-478 (backward kernel :127-254: the
//                 preactivation is recomputed into a buffer of x's dtype, then
//                 g = dy * s * (1 + y (1 - s)), dx = sum_j w_j g_{t+W-1-j}, dw partials per
//                 (batch, 64-token block) summed in order)
//   gated norm    FLA FusedRMSNormGated(D, activation="sigmoid", eps) as lit_gpt/iso_kdn.py:192-196,
//                 305-312 and lit_gpt/diag_kdn.py:216-219,346:
//                 y = x rsqrt(mean x^2 + eps) * w * act(g), act = sigmoid (or swish: g sigmoid(g))
#include <algorithm>

#include "kdn_common.h"
#include "../../include/kdn.h"

namespace {

constexpr int kConvW = 4;       // kernel width (the reference requires 4)
constexpr int kConvRun = 8;     // tokens per inner run of a thread
constexpr int kConvBlockT = 64; // tokens per backward thread (one dw partial per 64-token block)

template <typename T>
__device__ __forceinline__ void ld8v(const T* p, float* f);
template <>
__device__ __forceinline__ void ld8v<bf16_t>(const bf16_t* p, float* f) {
  const uint4 w = *reinterpret_cast<const uint4*>(p);
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    f[2 * q] = __uint_as_float(ww[q] << 16);
    f[2 * q + 1] = __uint_as_float(ww[q] & 0xffff0000u);
  }
}
template <>
__device__ __forceinline__ void ld8v<float>(const float* p, float* f) {
  const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
  f[0] = a.x, f[1] = a.y, f[2] = a.z, f[3] = a.w, f[4] = b.x, f[5] = b.y, f[6] = b.z, f[7] = b.w;
}
template <typename T>
__device__ __forceinline__ void st8v(T* p, const float* f);
template <>
__device__ __forceinline__ void st8v<bf16_t>(bf16_t* p, const float* f) {
  uint32_t w[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) w[q] = (uint32_t)f2bf(f[2 * q]) | ((uint32_t)f2bf(f[2 * q + 1]) << 16);
  *reinterpret_cast<uint4*>(p) = uint4{w[0], w[1], w[2], w[3]};
}
template <>
__device__ __forceinline__ void st8v<float>(float* p, const float* f) {
  reinterpret_cast<float4*>(p)[0] = float4{f[0], f[1], f[2], f[3]};
  reinterpret_cast<float4*>(p)[1] = float4{f[4], f[5], f[6], f[7]};
}
// value as stored in a buffer of type T (bf16 rounds to nearest even)
template <typename T>
__device__ __forceinline__ float as_stored(float x) {
  if constexpr (sizeof(T) == 2) return bf2f(f2bf(x));
  else return x;
}
template <typename T>
__device__ __forceinline__ float ld1(const T* p) {
  if constexpr (sizeof(T) == 2) return bf2f(*p);
  else return *p;
}
template <typename T>
__device__ __forceinline__ void st1(T* p, float x) {
  if constexpr (sizeof(T) == 2) *p = f2bf(x);
  else *p = x;
}
// weights of 8 consecutive channels x kConvW taps (row-major [D][W]): 32 contiguous elements
template <typename TW>
__device__ __forceinline__ void ld_taps(const TW* p, float (&wt)[8][kConvW]) {
  float f[32];
#pragma unroll
  for (int q = 0; q < 4; ++q) ld8v(p + 8 * q, f + 8 * q);
#pragma unroll
  for (int c = 0; c < 8; ++c)
#pragma unroll
    for (int j = 0; j < kConvW; ++j) wt[c][j] = f[c * kConvW + j];
}
// 8 channels of row t, or zeros outside [0, T): the load is unconditional (row clamped), so the
// compiler issues every row's load before the first use
template <typename TX>
__device__ __forceinline__ void ld_row(const TX* base, int64_t st, int t, int T, float* f) {
  const int tc = t < 0 ? 0 : (t >= T ? T - 1 : t);
  ld8v(base + (int64_t)tc * st, f);
  const bool ok = t >= 0 && t < T;
#pragma unroll
  for (int c = 0; c < 8; ++c) f[c] = ok ? f[c] : 0.f;
}
__device__ __forceinline__ float silu_grad(float y) {  // d/dy [y sigmoid(y)]
  const float s = sigmoidf(y);
  return s * (1.f + y * (1.f - s));
}

// ---------------------------------------------------------------------------
// Short convolution forward.  Thread = (b, 8-token run, 8-channel group), channel groups
// fastest.  y_t = silu(sum_j w_j x_{t-3+j}), x_{<0} = 0, fp32 then rounded to y's dtype.
// ---------------------------------------------------------------------------
template <typename TX, typename TW>
__global__ __launch_bounds__(256) void short_conv_fwd_kernel(const TX* __restrict__ x, int64_t xsb, int64_t xst,
                                                             const TW* __restrict__ w, int B, int T, int D,
                                                             TX* __restrict__ y, int64_t ysb, int64_t yst) {
  const int CG = D / 8, NR = (T + kConvRun - 1) / kConvRun;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (int64_t)B * NR * CG) return;
  const int cg = (int)(gid % CG), run = (int)((gid / CG) % NR), b = (int)(gid / ((int64_t)CG * NR));
  const int d0 = 8 * cg, t0 = run * kConvRun;
  float wt[8][kConvW];
  ld_taps(w + (int64_t)d0 * kConvW, wt);
  constexpr int NX = kConvRun + kConvW - 1;
  float xr[NX][8];
#pragma unroll
  for (int r = 0; r < NX; ++r) ld_row(x + (int64_t)b * xsb + d0, xst, t0 - (kConvW - 1) + r, T, xr[r]);
#pragma unroll
  for (int u = 0; u < kConvRun; ++u) {
    const int t = t0 + u;
    if (t >= T) break;
    float o[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float a = 0.f;
#pragma unroll
      for (int j = 0; j < kConvW; ++j) a += wt[c][j] * xr[u + j][c];
      o[c] = a * sigmoidf(a);
    }
    st8v(y + (int64_t)b * ysb + (int64_t)t * yst + d0, o);
  }
}

// ---------------------------------------------------------------------------
// One token of the short convolution with its carried inputs (decoding): thread = (b, 8 channels).
// y = silu(w_0 s_0 + w_1 s_1 + w_2 s_2 + w_3 x) with s the 3 earlier inputs (tail [B,3,D], x's
// dtype), summed in the order of short_conv_fwd_kernel, so it equals that kernel run over
// [s, x]; then the tail shifts in place to [s_1, s_2, x].  Each thread reads its own channels'
// tail before writing them.
// ---------------------------------------------------------------------------
template <typename TX, typename TW>
__global__ __launch_bounds__(256) void short_conv_step_kernel(const TX* __restrict__ x, int64_t xsb,
                                                              TX* __restrict__ tail, int64_t tsb,
                                                              const TW* __restrict__ w, int B, int D,
                                                              TX* __restrict__ y, int64_t ysb) {
  const int CG = D / 8;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (int64_t)B * CG) return;
  const int cg = (int)(gid % CG), b = (int)(gid / CG), d0 = 8 * cg;
  float wt[8][kConvW];
  ld_taps(w + (int64_t)d0 * kConvW, wt);
  float xr[kConvW][8];
  TX* tb = tail + (int64_t)b * tsb + d0;
#pragma unroll
  for (int r = 0; r < kConvW - 1; ++r) ld8v(tb + (int64_t)r * D, xr[r]);
  ld8v(x + (int64_t)b * xsb + d0, xr[kConvW - 1]);
  float o[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    float a = 0.f;
#pragma unroll
    for (int j = 0; j < kConvW; ++j) a += wt[c][j] * xr[j][c];
    o[c] = a * sigmoidf(a);
  }
  st8v(y + (int64_t)b * ysb + d0, o);
#pragma unroll
  for (int r = 0; r < kConvW - 1; ++r) st8v(tb + (int64_t)r * D, xr[r + 1]);  // exact: values of TX
}

// ---------------------------------------------------------------------------
// Short convolution backward.  Block = 32 channel groups x 8 runs of 8 tokens (one 64-token
// block of 256 channels); thread = (run, channel group), all its loads issued at once.
// g_t = dy_t silu'(y_t) with y the recomputed preactivation (rounded to x's dtype when round_y,
// as the reference's raw_y buffer is), dx_t = sum_j w_j g_{t+3-j}, and the dw_j partial
// sum_t g_t x_{t-3+j} over the 64 tokens, reduced over the runs in LDS in a fixed order
// -> part[b * NB + blk][d][j].
// ---------------------------------------------------------------------------
constexpr int kConvCG = 32;  // channel groups per backward block
template <typename TX, typename TW>
__global__ __launch_bounds__(256) void short_conv_bwd_kernel(const TX* __restrict__ x, int64_t xsb, int64_t xst,
                                                             const TW* __restrict__ w, const TX* __restrict__ dy,
                                                             int64_t dsb, int64_t dst, int B, int T, int D,
                                                             int round_y, TX* __restrict__ dx, int64_t gsb,
                                                             int64_t gst, float* __restrict__ part) {
  __shared__ float s_dw[kConvBlockT / kConvRun][kConvCG * 8 * kConvW];
  const int CG = D / 8, NB = (T + kConvBlockT - 1) / kConvBlockT, NCB = (CG + kConvCG - 1) / kConvCG;
  const int cb = blockIdx.x % NCB, blk = (blockIdx.x / NCB) % NB, b = blockIdx.x / (NCB * NB);
  const int lc = threadIdx.x % kConvCG, run = threadIdx.x / kConvCG;
  const int cg = cb * kConvCG + lc, d0 = 8 * cg, t0 = blk * kConvBlockT + run * kConvRun;
  const bool active = cg < CG && t0 < T;
  float dw[8][kConvW];
#pragma unroll
  for (int c = 0; c < 8; ++c)
#pragma unroll
    for (int j = 0; j < kConvW; ++j) dw[c][j] = 0.f;
  if (active) {
    float wt[8][kConvW];
    ld_taps(w + (int64_t)d0 * kConvW, wt);
    constexpr int NX = kConvRun + 2 * (kConvW - 1);  // x rows t0-3 .. t0+run+2
    constexpr int NG = kConvRun + kConvW - 1;        // g at t0 .. t0+run+2
    float xr[NX][8], dyr[NG][8];
#pragma unroll
    for (int r = 0; r < NX; ++r) ld_row(x + (int64_t)b * xsb + d0, xst, t0 - (kConvW - 1) + r, T, xr[r]);
    if (dy) {
#pragma unroll
      for (int r = 0; r < NG; ++r) ld_row(dy + (int64_t)b * dsb + d0, dst, t0 + r, T, dyr[r]);
    } else {
#pragma unroll
      for (int r = 0; r < NG; ++r)
#pragma unroll
        for (int c = 0; c < 8; ++c) dyr[r][c] = 0.f;
    }
    float gr[NG][8];
#pragma unroll
    for (int r = 0; r < NG; ++r)
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        float a = 0.f;
#pragma unroll
        for (int j = 0; j < kConvW; ++j) a += wt[c][j] * xr[r + j][c];
        if (round_y) a = as_stored<TX>(a);
        gr[r][c] = dyr[r][c] * silu_grad(a);
      }
#pragma unroll
    for (int u = 0; u < kConvRun; ++u) {
      const int t = t0 + u;
      if (t >= T) break;
      float o[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        float a = 0.f;
#pragma unroll
        for (int j = 0; j < kConvW; ++j) a += wt[c][j] * gr[u + kConvW - 1 - j][c];
        o[c] = a;
#pragma unroll
        for (int j = 0; j < kConvW; ++j) dw[c][j] += gr[u][c] * xr[u + j][c];
      }
      if (dx) st8v(dx + (int64_t)b * gsb + (int64_t)t * gst + d0, o);
    }
  }
  if (!part) return;
  // [run][tap][channel-in-group][group]: consecutive lanes (groups) hit consecutive banks
#pragma unroll
  for (int c = 0; c < 8; ++c)
#pragma unroll
    for (int j = 0; j < kConvW; ++j) s_dw[run][(j * 8 + c) * kConvCG + lc] = dw[c][j];
  __syncthreads();
  // this block's 256 channels x 4 taps, summed over the 8 runs in order
  for (int e = threadIdx.x; e < kConvCG * 8 * kConvW; e += 256) {
    const int q = e / kConvW, j = e % kConvW;  // q = local channel (group-major), j = tap
    const int lg = q / 8, c = q % 8, d = cb * kConvCG * 8 + q;
    if (d >= D) continue;
    float acc = 0.f;
#pragma unroll
    for (int r = 0; r < kConvBlockT / kConvRun; ++r) acc += s_dw[r][(j * 8 + c) * kConvCG + lg];
    part[((int64_t)b * NB + blk) * D * kConvW + (int64_t)d * kConvW + j] = acc;
  }
}

// out[j] = sum_p part[p * n + j] in a fixed order: block = 16 columns x 16 stripes of p, the
// stripes combined by a fixed LDS tree.  grid ceil(n/16).
template <typename TO>
__global__ __launch_bounds__(256) void sum_partials_kernel(const float* __restrict__ part, int NP, int64_t n,
                                                           TO* __restrict__ out) {
  __shared__ float s[16][17];
  const int jj = threadIdx.x & 15, st = threadIdx.x >> 4;
  const int64_t j = (int64_t)blockIdx.x * 16 + jj;
  float a0 = 0.f, a1 = 0.f;
  if (j < n) {
    int p = st;
    for (; p + 16 < NP; p += 32) a0 += part[(int64_t)p * n + j], a1 += part[(int64_t)(p + 16) * n + j];
    for (; p < NP; p += 16) a0 += part[(int64_t)p * n + j];
  }
  s[st][jj] = a0 + a1;
  __syncthreads();
  for (int h = 8; h > 0; h >>= 1) {
    if (st < h) s[st][jj] += s[st + h][jj];
    __syncthreads();
  }
  if (st == 0 && j < n) st1(out + j, s[0][jj]);
}

// ---------------------------------------------------------------------------
// Gated RMS norm.  D/8 lanes per row, 8 elements per lane, 256/(D/8) rows per block.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float row_sum(float v, int lanes) {
  for (int o = 1; o < lanes; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float gate_act(float g, int act) {  // 0: sigmoid(g), 1: g sigmoid(g)
  const float s = sigmoidf(g);
  return act == 0 ? s : g * s;
}
__device__ __forceinline__ float gate_grad(float g, int act) {
  const float s = sigmoidf(g);
  return act == 0 ? s * (1.f - s) : s * (1.f + g * (1.f - s));
}

template <typename TX, typename TG, typename TW>
__global__ __launch_bounds__(256) void rms_gated_fwd_kernel(const TX* __restrict__ x, const TG* __restrict__ g,
                                                            const TW* __restrict__ w, int64_t rows, int D, float eps,
                                                            int act, TX* __restrict__ y, float* __restrict__ rstd) {
  const int LPR = D / 8, RPB = 256 / LPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR;
  const int sub = threadIdx.x % LPR, d0 = 8 * sub;
  float xv[8], gv[8], wv[8], ss = 0.f;
  const bool ok = row < rows;
  const int64_t rr = ok ? row : 0;
  ld8v(x + rr * D + d0, xv);
  ld8v(g + rr * D + d0, gv);
  ld8v(w + d0, wv);
#pragma unroll
  for (int c = 0; c < 8; ++c) ss += xv[c] * xv[c];
  ss = row_sum(ss, LPR);
  const float rs = rsqrtf(ss / (float)D + eps);
  float o[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) o[c] = xv[c] * rs * wv[c] * gate_act(gv[c], act);
  if (!ok) return;
  st8v(y + row * D + d0, o);
  if (sub == 0 && rstd) rstd[row] = rs;
}

// Backward: grid-stride over row groups with a fixed grid; each thread accumulates its 8
// channels' dweight over its rows, then the block sums its row slots in order -> part[block][D].
constexpr int kRmsBwdBlocks = 1024;
template <typename TX, typename TG, typename TW>
__global__ __launch_bounds__(256) void rms_gated_bwd_kernel(const TX* __restrict__ x, const TG* __restrict__ g,
                                                            const TW* __restrict__ w, const float* __restrict__ rstd,
                                                            const TX* __restrict__ dy, int64_t rows, int D, int act,
                                                            TX* __restrict__ dx, TG* __restrict__ dg,
                                                            float* __restrict__ part) {
  __shared__ float s_dw[256 * 8];
  const int LPR = D / 8, RPB = 256 / LPR;
  const int r_in = threadIdx.x / LPR;
  const int sub = threadIdx.x % LPR, d0 = 8 * sub;
  float wv[8], dwv[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) dwv[c] = 0.f;
  ld8v(w + d0, wv);
  for (int64_t base = (int64_t)blockIdx.x * RPB; base < rows; base += (int64_t)gridDim.x * RPB) {
    const int64_t row = base + r_in;
    const bool ok = row < rows;
    const int64_t rr = ok ? row : 0;
    float xv[8], gv[8], dyv[8];
    ld8v(x + rr * D + d0, xv);
    ld8v(g + rr * D + d0, gv);
    ld8v(dy + rr * D + d0, dyv);
    const float rs = rstd[rr];
    float dn[8], n[8], av[8], dot = 0.f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      n[c] = xv[c] * rs;
      av[c] = gate_act(gv[c], act);
      dn[c] = dyv[c] * wv[c] * av[c];
      dot += dn[c] * n[c];
    }
    dot = row_sum(dot, LPR) / (float)D;
    if (ok) {
      float o[8], og[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        o[c] = rs * (dn[c] - n[c] * dot);
        og[c] = dyv[c] * n[c] * wv[c] * gate_grad(gv[c], act);
        dwv[c] += dyv[c] * n[c] * av[c];
      }
      if (dx) st8v(dx + row * D + d0, o);
      if (dg) st8v(dg + row * D + d0, og);
    }
  }
  if (!part) return;
#pragma unroll
  for (int c = 0; c < 8; ++c) s_dw[r_in * D + d0 + c] = dwv[c];
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += 256) {
    float s = 0.f;
    for (int q = 0; q < RPB; ++q) s += s_dw[q * D + d];
    part[(int64_t)blockIdx.x * D + d] = s;
  }
}

// ---------------------------------------------------------------------------
// Block RMS norm over wide rows (the model's FusedRMSNorm, D = n_embd): one workgroup per row,
// 8 elements per thread per pass, block sum through LDS.  y = x rsqrt(mean x^2 + eps) * w.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float block_sum256(float v, float* red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

template <typename TX, typename TW>
__global__ __launch_bounds__(256) void rms_row_fwd_kernel(const TX* __restrict__ x, const TW* __restrict__ w, int D,
                                                          float eps, TX* __restrict__ y, float* __restrict__ rstd) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const TX* xr = x + row * D;
  float ss = 0.f;
  for (int d0 = 8 * threadIdx.x; d0 < D; d0 += 8 * 256) {
    float v[8];
    ld8v(xr + d0, v);
#pragma unroll
    for (int c = 0; c < 8; ++c) ss += v[c] * v[c];
  }
  const float rs = rsqrtf(block_sum256(ss, red) / (float)D + eps);
  for (int d0 = 8 * threadIdx.x; d0 < D; d0 += 8 * 256) {
    float v[8], wv[8];
    ld8v(xr + d0, v);
    ld8v(w + d0, wv);
#pragma unroll
    for (int c = 0; c < 8; ++c) v[c] = v[c] * rs * wv[c];
    st8v(y + row * D + d0, v);
  }
  if (threadIdx.x == 0 && rstd) rstd[row] = rs;
}

// backward: dx = rstd (dy w - n mean(dy w n)), n = x rstd; dweight partial per workgroup
// (one row) accumulated over a fixed stride of rows: part[blockIdx.x][D]
template <typename TX, typename TW>
__global__ __launch_bounds__(256) void rms_row_bwd_kernel(const TX* __restrict__ x, const TW* __restrict__ w,
                                                          const float* __restrict__ rstd, const TX* __restrict__ dy,
                                                          int64_t rows, int D, TX* __restrict__ dx,
                                                          float* __restrict__ part) {
  __shared__ float red[4];
  constexpr int MAXG = 4;  // up to 4 passes of 2048 elements per thread-slot: D <= 8192
  float dwv[MAXG][8];
#pragma unroll
  for (int q = 0; q < MAXG; ++q)
#pragma unroll
    for (int c = 0; c < 8; ++c) dwv[q][c] = 0.f;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const float rs = rstd[row];
    float dot = 0.f;
#pragma unroll
    for (int q = 0; q < MAXG; ++q) {
      const int d0 = 8 * threadIdx.x + 2048 * q;
      if (d0 >= D) break;
      float xv[8], dv[8], wv[8];
      ld8v(x + row * D + d0, xv);
      ld8v(dy + row * D + d0, dv);
      ld8v(w + d0, wv);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const float n = xv[c] * rs;
        dot += dv[c] * wv[c] * n;
        dwv[q][c] += dv[c] * n;
      }
    }
    dot = block_sum256(dot, red) / (float)D;
    if (dx) {
#pragma unroll
      for (int q = 0; q < MAXG; ++q) {
        const int d0 = 8 * threadIdx.x + 2048 * q;
        if (d0 >= D) break;
        float xv[8], dv[8], wv[8], o[8];
        ld8v(x + row * D + d0, xv);
        ld8v(dy + row * D + d0, dv);
        ld8v(w + d0, wv);
#pragma unroll
        for (int c = 0; c < 8; ++c) o[c] = rs * (dv[c] * wv[c] - xv[c] * rs * dot);
        st8v(dx + row * D + d0, o);
      }
    }
  }
  if (!part) return;
#pragma unroll
  for (int q = 0; q < MAXG; ++q) {
    const int d0 = 8 * threadIdx.x + 2048 * q;
    if (d0 >= D) break;
    st8v(part + (int64_t)blockIdx.x * D + d0, dwv[q]);
  }
}
constexpr int kRmsRowBwdBlocks = 512;

bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

extern "C" {

// ---------------------------------------------------------------------------------- short conv
int kdn_short_conv_fwd(const void* x, int x_bf16, int64_t x_stride_b, int64_t x_stride_t, const void* weight,
                       int w_bf16, int B, int T, int D, int W, void* y, int64_t y_stride_b, int64_t y_stride_t,
                       hipStream_t stream) {
  if (B < 0 || T < 0 || D <= 0 || W != kConvW || D % 8 != 0 || !x || !weight || !y) return KDN_ERR_ARG;
  if (!al16(x) || !al16(y) || !al16(weight) || x_stride_t % 8 != 0 || x_stride_b % 8 != 0 || y_stride_t % 8 != 0 ||
      y_stride_b % 8 != 0)
    return KDN_ERR_ARG;
  if (B == 0 || T == 0) return 0;
  const int64_t threads = (int64_t)B * ((T + kConvRun - 1) / kConvRun) * (D / 8);
  const dim3 grid((unsigned)((threads + 255) / 256));
#define KDN_CONV_FWD(TX, TW)                                                                                         \
  hipLaunchKernelGGL((short_conv_fwd_kernel<TX, TW>), grid, dim3(256), 0, stream, (const TX*)x, x_stride_b,         \
                     x_stride_t, (const TW*)weight, B, T, D, (TX*)y, y_stride_b, y_stride_t)
  if (x_bf16 && w_bf16) KDN_CONV_FWD(bf16_t, bf16_t);
  else if (x_bf16) KDN_CONV_FWD(bf16_t, float);
  else if (w_bf16) KDN_CONV_FWD(float, bf16_t);
  else KDN_CONV_FWD(float, float);
#undef KDN_CONV_FWD
  KDN_CHECK_LAUNCH();
  return 0;
}

int kdn_short_conv_step(const void* x, int x_bf16, int64_t x_stride_b, void* tail, int64_t tail_stride_b,
                        const void* weight, int w_bf16, int B, int D, void* y, int64_t y_stride_b,
                        hipStream_t stream) {
  if (B < 0 || D <= 0 || D % 8 != 0 || !x || !tail || !weight || !y) return KDN_ERR_ARG;
  // batch strides are used only for B > 1; they keep every row 16-byte aligned
  if (!al16(x) || !al16(y) || !al16(tail) || !al16(weight) || tail_stride_b < (int64_t)(kConvW - 1) * D)
    return KDN_ERR_ARG;
  if (B > 1 && (x_stride_b % 8 != 0 || y_stride_b % 8 != 0 || tail_stride_b % 8 != 0)) return KDN_ERR_ARG;
  if (B == 0) return 0;
  const int64_t threads = (int64_t)B * (D / 8);
  const dim3 grid((unsigned)((threads + 255) / 256));
#define KDN_CONV_STEP(TX, TW)                                                                                        \
  hipLaunchKernelGGL((short_conv_step_kernel<TX, TW>), grid, dim3(256), 0, stream, (const TX*)x, x_stride_b,        \
                     (TX*)tail, tail_stride_b, (const TW*)weight, B, D, (TX*)y, y_stride_b)
  if (x_bf16 && w_bf16) KDN_CONV_STEP(bf16_t, bf16_t);
  else if (x_bf16) KDN_CONV_STEP(bf16_t, float);
  else if (w_bf16) KDN_CONV_STEP(float, bf16_t);
  else KDN_CONV_STEP(float, float);
#undef KDN_CONV_STEP
  KDN_CHECK_LAUNCH();
  return 0;
}

size_t kdn_short_conv_bwd_workspace_size(int B, int T, int D) {
  if (B <= 0 || T <= 0 || D <= 0) return 0;
  const int64_t NB = (T + kConvBlockT - 1) / kConvBlockT;
  return (size_t)((int64_t)B * NB * D * kConvW) * sizeof(float);
}

int kdn_short_conv_bwd(const void* x, int x_bf16, int64_t x_stride_b, int64_t x_stride_t, const void* weight,
                       int w_bf16, const void* dy, int64_t dy_stride_b, int64_t dy_stride_t, int B, int T, int D,
                       int W, int round_preactivation, void* dx, int64_t dx_stride_b, int64_t dx_stride_t,
                       void* dweight, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (B < 0 || T < 0 || D <= 0 || W != kConvW || D % 8 != 0 || !x || !weight) return KDN_ERR_ARG;
  if (!al16(x) || !al16(weight) || (dy && !al16(dy)) || (dx && !al16(dx)) || x_stride_t % 8 || x_stride_b % 8 ||
      (dy && (dy_stride_t % 8 || dy_stride_b % 8)) || (dx && (dx_stride_t % 8 || dx_stride_b % 8)))
    return KDN_ERR_ARG;
  if (B == 0 || T == 0) return 0;
  if (dweight && (!workspace || workspace_bytes < kdn_short_conv_bwd_workspace_size(B, T, D) ||
                  !al16(workspace)))
    return KDN_ERR_ARG;
  const int NB = (T + kConvBlockT - 1) / kConvBlockT, NCB = (D / 8 + kConvCG - 1) / kConvCG;
  const dim3 grid((unsigned)((int64_t)B * NB * NCB));
  float* part = dweight ? (float*)workspace : nullptr;
  if (!dweight && !dx) return 0;
#define KDN_CONV_BWD(TX, TW)                                                                                       \
  hipLaunchKernelGGL((short_conv_bwd_kernel<TX, TW>), grid, dim3(256), 0, stream, (const TX*)x, x_stride_b,       \
                     x_stride_t, (const TW*)weight, (const TX*)dy, dy_stride_b, dy_stride_t, B, T, D,             \
                     round_preactivation, (TX*)dx, dx_stride_b, dx_stride_t, part)
  if (x_bf16 && w_bf16) KDN_CONV_BWD(bf16_t, bf16_t);
  else if (x_bf16) KDN_CONV_BWD(bf16_t, float);
  else if (w_bf16) KDN_CONV_BWD(float, bf16_t);
  else KDN_CONV_BWD(float, float);
#undef KDN_CONV_BWD
  KDN_CHECK_LAUNCH();
  if (dweight) {
    const int64_t n = (int64_t)D * kConvW;
    const dim3 rg((unsigned)((n + 15) / 16));
    if (w_bf16)
      hipLaunchKernelGGL((sum_partials_kernel<bf16_t>), rg, dim3(256), 0, stream, part, B * NB, n, (bf16_t*)dweight);
    else
      hipLaunchKernelGGL((sum_partials_kernel<float>), rg, dim3(256), 0, stream, part, B * NB, n, (float*)dweight);
    KDN_CHECK_LAUNCH();
  }
  return 0;
}

// ---------------------------------------------------------------------------------- gated norm
static bool rms_shape_ok(int D) { return D % 8 == 0 && D / 8 <= 64 && (D / 8 & (D / 8 - 1)) == 0; }

// ---------------------------------------------------------------------------------- block RMS norm
int kdn_rms_norm_fwd(const void* x, int x_bf16, const void* weight, int w_bf16, int64_t rows, int D, float eps,
                     void* y, float* rstd, hipStream_t stream) {
  if (rows < 0 || D <= 0 || D % 8 != 0 || D > 8192 || !(eps >= 0.f)) return KDN_ERR_ARG;
  if (!x || !weight || !y || !al16(x) || !al16(weight) || !al16(y)) return KDN_ERR_ARG;
  if (rows == 0) return 0;
  const dim3 grid((unsigned)rows);
#define KDN_ROW_FWD(TX, TW)                                                                                        \
  hipLaunchKernelGGL((rms_row_fwd_kernel<TX, TW>), grid, dim3(256), 0, stream, (const TX*)x, (const TW*)weight, D, \
                     eps, (TX*)y, rstd)
  if (x_bf16) { if (w_bf16) KDN_ROW_FWD(bf16_t, bf16_t); else KDN_ROW_FWD(bf16_t, float); }
  else { if (w_bf16) KDN_ROW_FWD(float, bf16_t); else KDN_ROW_FWD(float, float); }
#undef KDN_ROW_FWD
  KDN_CHECK_LAUNCH();
  return 0;
}

size_t kdn_rms_norm_bwd_workspace_size(int64_t rows, int D) {
  if (rows <= 0 || D <= 0) return 0;
  return (size_t)(std::min<int64_t>(rows, kRmsRowBwdBlocks) * D) * sizeof(float);
}

int kdn_rms_norm_bwd(const void* x, int x_bf16, const void* weight, int w_bf16, const float* rstd, const void* dy,
                     int64_t rows, int D, void* dx, void* dweight, void* workspace, size_t workspace_bytes,
                     hipStream_t stream) {
  if (rows < 0 || D <= 0 || D % 8 != 0 || D > 8192) return KDN_ERR_ARG;
  if (!x || !weight || !rstd || !dy || !al16(x) || !al16(weight) || !al16(dy) || (dx && !al16(dx)))
    return KDN_ERR_ARG;
  if (rows == 0) return 0;
  if (dweight && (!workspace || workspace_bytes < kdn_rms_norm_bwd_workspace_size(rows, D) || !al16(workspace)))
    return KDN_ERR_ARG;
  const int NBLK = (int)std::min<int64_t>(rows, kRmsRowBwdBlocks);
  float* part = dweight ? (float*)workspace : nullptr;
#define KDN_ROW_BWD(TX, TW)                                                                                       \
  hipLaunchKernelGGL((rms_row_bwd_kernel<TX, TW>), dim3(NBLK), dim3(256), 0, stream, (const TX*)x,               \
                     (const TW*)weight, rstd, (const TX*)dy, rows, D, (TX*)dx, part)
  if (x_bf16) { if (w_bf16) KDN_ROW_BWD(bf16_t, bf16_t); else KDN_ROW_BWD(bf16_t, float); }
  else { if (w_bf16) KDN_ROW_BWD(float, bf16_t); else KDN_ROW_BWD(float, float); }
#undef KDN_ROW_BWD
  KDN_CHECK_LAUNCH();
  if (dweight) {
    const dim3 rg((unsigned)((D + 15) / 16));
    if (w_bf16)
      hipLaunchKernelGGL((sum_partials_kernel<bf16_t>), rg, dim3(256), 0, stream, part, NBLK, (int64_t)D, (bf16_t*)dweight);
    else
      hipLaunchKernelGGL((sum_partials_kernel<float>), rg, dim3(256), 0, stream, part, NBLK, (int64_t)D, (float*)dweight);
    KDN_CHECK_LAUNCH();
  }
  return 0;
}

int kdn_rms_norm_gated_fwd(const void* x, int x_bf16, const void* g, int g_bf16, const void* weight, int w_bf16,
                           int64_t rows, int D, float eps, int activation, void* y, float* rstd,
                           hipStream_t stream) {
  if (rows < 0 || D <= 0 || !rms_shape_ok(D) || (activation != 0 && activation != 1) || !(eps >= 0.f)) return KDN_ERR_ARG;
  if (!x || !g || !weight || !y || !al16(x) || !al16(g) || !al16(y) || !al16(weight)) return KDN_ERR_ARG;
  if (rows == 0) return 0;
  const int RPB = 256 / (D / 8);
  const dim3 grid((unsigned)((rows + RPB - 1) / RPB));
#define KDN_RMS_FWD(TX, TG, TW)                                                                                   \
  hipLaunchKernelGGL((rms_gated_fwd_kernel<TX, TG, TW>), grid, dim3(256), 0, stream, (const TX*)x, (const TG*)g, \
                     (const TW*)weight, rows, D, eps, activation, (TX*)y, rstd)
  if (x_bf16) {
    if (g_bf16) { if (w_bf16) KDN_RMS_FWD(bf16_t, bf16_t, bf16_t); else KDN_RMS_FWD(bf16_t, bf16_t, float); }
    else { if (w_bf16) KDN_RMS_FWD(bf16_t, float, bf16_t); else KDN_RMS_FWD(bf16_t, float, float); }
  } else {
    if (g_bf16) { if (w_bf16) KDN_RMS_FWD(float, bf16_t, bf16_t); else KDN_RMS_FWD(float, bf16_t, float); }
    else { if (w_bf16) KDN_RMS_FWD(float, float, bf16_t); else KDN_RMS_FWD(float, float, float); }
  }
#undef KDN_RMS_FWD
  KDN_CHECK_LAUNCH();
  return 0;
}

size_t kdn_rms_norm_gated_bwd_workspace_size(int64_t rows, int D) {
  if (rows <= 0 || D <= 0 || !rms_shape_ok(D)) return 0;
  const int RPB = 256 / (D / 8);
  const int64_t nblk = std::min<int64_t>((rows + RPB - 1) / RPB, kRmsBwdBlocks);
  return (size_t)(nblk * D) * sizeof(float);
}

int kdn_rms_norm_gated_bwd(const void* x, int x_bf16, const void* g, int g_bf16, const void* weight, int w_bf16,
                           const float* rstd, const void* dy, int64_t rows, int D, int activation, void* dx,
                           void* dg, void* dweight, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (rows < 0 || D <= 0 || !rms_shape_ok(D) || (activation != 0 && activation != 1)) return KDN_ERR_ARG;
  if (!x || !g || !weight || !rstd || !dy || !al16(x) || !al16(g) || !al16(dy) || !al16(weight) || (dx && !al16(dx)) ||
      (dg && !al16(dg)))
    return KDN_ERR_ARG;
  if (rows == 0) return 0;
  if (dweight && (!workspace || workspace_bytes < kdn_rms_norm_gated_bwd_workspace_size(rows, D))) return KDN_ERR_ARG;
  const int RPB = 256 / (D / 8);
  const int NBLK = (int)std::min<int64_t>((rows + RPB - 1) / RPB, kRmsBwdBlocks);
  float* part = dweight ? (float*)workspace : nullptr;
#define KDN_RMS_BWD(TX, TG, TW)                                                                                     \
  hipLaunchKernelGGL((rms_gated_bwd_kernel<TX, TG, TW>), dim3(NBLK), dim3(256), 0, stream, (const TX*)x,           \
                     (const TG*)g, (const TW*)weight, rstd, (const TX*)dy, rows, D, activation, (TX*)dx, (TG*)dg,   \
                     part)
  if (x_bf16) {
    if (g_bf16) { if (w_bf16) KDN_RMS_BWD(bf16_t, bf16_t, bf16_t); else KDN_RMS_BWD(bf16_t, bf16_t, float); }
    else { if (w_bf16) KDN_RMS_BWD(bf16_t, float, bf16_t); else KDN_RMS_BWD(bf16_t, float, float); }
  } else {
    if (g_bf16) { if (w_bf16) KDN_RMS_BWD(float, bf16_t, bf16_t); else KDN_RMS_BWD(float, bf16_t, float); }
    else { if (w_bf16) KDN_RMS_BWD(float, float, bf16_t); else KDN_RMS_BWD(float, float, float); }
  }
#undef KDN_RMS_BWD
  KDN_CHECK_LAUNCH();
  if (dweight) {
    const dim3 rg((unsigned)((D + 15) / 16));
    if (w_bf16)
      hipLaunchKernelGGL((sum_partials_kernel<bf16_t>), rg, dim3(256), 0, stream, part, NBLK, (int64_t)D, (bf16_t*)dweight);
    else
      hipLaunchKernelGGL((sum_partials_kernel<float>), rg, dim3(256), 0, stream, part, NBLK, (int64_t)D, (float*)dweight);
    KDN_CHECK_LAUNCH();
  }
  return 0;
}

}  // extern "C"
