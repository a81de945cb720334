// Shared device helpers for the KDN HIP kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "kdn.h"

#define KDN_LN2 0.6931471805599453f
#define KDN_LOG2E 1.4426950408889634f

typedef uint16_t bf16_t;  // raw bfloat16 bits
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ---- bf16 <-> fp32 ----------------------------------------------------------
__device__ __forceinline__ float bf2f(bf16_t u) { return __uint_as_float(((uint32_t)u) << 16); }
// round to nearest even (NaN stays NaN): gfx950's v_cvt_pk_bf16_f32, one instruction for two values
__device__ __forceinline__ bf16_t f2bf(float x) { return __builtin_bit_cast(bf16_t, (__bf16)x); }

template <typename T> __device__ __forceinline__ float ld(const T* p, int64_t i);
template <> __device__ __forceinline__ float ld<float>(const float* p, int64_t i) { return p[i]; }
template <> __device__ __forceinline__ float ld<bf16_t>(const bf16_t* p, int64_t i) { return bf2f(p[i]); }
template <typename T> __device__ __forceinline__ void st(T* p, int64_t i, float x);
template <> __device__ __forceinline__ void st<float>(float* p, int64_t i, float x) { p[i] = x; }
template <> __device__ __forceinline__ void st<bf16_t>(bf16_t* p, int64_t i, float x) { p[i] = f2bf(x); }

// ---- buffer-descriptor memory access ----------------------------------------------
// A raw buffer descriptor over [base, base + bytes) (gfx9 dword3: 32-bit data format).
// Loads at or past `bytes` return 0 and stores there are dropped, which replaces
// per-element bounds branches; offsets are 32-bit bytes.  `base` must be wave-uniform.
typedef __amdgpu_buffer_rsrc_t bufrsrc;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ bufrsrc make_buf(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float buf_ld(bufrsrc r, uint32_t off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ float4 buf_ld4(bufrsrc r, uint32_t off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return float4{__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w)};
}
__device__ __forceinline__ float buf_ld_bf16(bufrsrc r, uint32_t off) {
  return bf2f(__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
}
template <typename T> __device__ __forceinline__ float buf_ldt(bufrsrc r, uint32_t elem);
template <> __device__ __forceinline__ float buf_ldt<float>(bufrsrc r, uint32_t elem) { return buf_ld(r, elem * 4); }
template <> __device__ __forceinline__ float buf_ldt<bf16_t>(bufrsrc r, uint32_t elem) {
  return buf_ld_bf16(r, elem * 2);
}
__device__ __forceinline__ void buf_st(bufrsrc r, uint32_t off, float x) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), r, off, 0, 0);
}

// ---- activations ---------------------------------------------------------------
// softplus with torch's default threshold (x > 20 -> x), on the hardware exp/log
// (v_exp_f32 / v_log_f32, a few ulp); log1p(y) = y (1 - y/2) below y = 1e-3 keeps small
// values accurate to ~y^3/3.
__device__ __forceinline__ float softplusf(float x) {
  if (x > 20.f) return x;
  const float y = __expf(x);
  return y < 1e-3f ? y * (1.f - 0.5f * y) : __logf(1.f + y);
}
__device__ __forceinline__ float sigmoidf(float x) { return __frcp_rn(1.f + __expf(-x)); }
// softplus(x) and sigmoid(x) from one exponential y = e^min(x, 20): softplus = x above 20 (torch's
// threshold), else log(1 + y) (y (1 - y/2) below y = 1e-3); sigmoid = y / (1 + y) with the hardware
// reciprocal (~1 ulp; it rounds to 1 above 20, as 1 / (1 + e^-x) does in fp32).
__device__ __forceinline__ void softplus_sigmoid(float x, float& sp, float& sg) {
  const float y = __expf(fminf(x, 20.f));
  const float d = 1.f + y;
  sg = y * __builtin_amdgcn_rcpf(d);
  sp = x > 20.f ? x : (y < 1e-3f ? y * (1.f - 0.5f * y) : __logf(d));
}

// Fast forms for kernels bound by vector-ALU issue: the hardware reciprocal (v_rcp_f32, 1 ulp; an IEEE
// division is about ten instructions), exp and log on v_exp_f32 / v_log_f32 (~1 ulp), and
// branch-free softplus / sigmoid.
__device__ __forceinline__ float frcp(float x) { return __builtin_amdgcn_rcpf(x); }
// exp and softplus on the hardware exp2 / log2 (one v_exp_f32 / v_log_f32 each, ~1 ulp), without
// branches: both sides of torch's threshold (x > 20 -> x) and of the small-value series are formed
// and selected, so no exec-mask branching sits in the token loops.  NaN propagates.
// The in-op L2 norm of the isotropic scan (FLA l2norm_fwd, iso_kdn_chunk.py:2203-2204): the scan
// consumes y = bf16(x rstd), rstd = 1 / sqrt(sum x^2 + 1e-6), per 128- or 64-channel row.  Kernels
// that take the raw bf16 q, k with their rows' rstd form y at the load with l2n; kdn_l2norm_fwd forms
// the same y (same expression, same rounding).
constexpr float kL2NormEps = 1e-6f;
__device__ __forceinline__ float l2n_rstd(float ss) { return 1.f / sqrtf(ss + kL2NormEps); }
__device__ __forceinline__ float l2n(float x, float rs) { return bf2f(f2bf(x * rs)); }
// The sum of squares of a row of 8 * NS channels given as NS runs of 8, in the order of
// l2norm_fwd_vec_kernel: each run summed in order, then the runs pairwise (run s with s ^ 1, then
// pairs of pairs, ...), the xor tree of its 8-channel lanes.  S[s] = sum of run s.
template <int NS>
__device__ __forceinline__ float l2n_tree(float* S) {
#pragma unroll
  for (int d = 1; d < NS; d <<= 1)
#pragma unroll
    for (int s = 0; s < NS; s += 2 * d) S[s] = S[s] + S[s + d];
  return S[0];
}
__device__ __forceinline__ float l2n_run(const float* x) {  // one run of 8, summed in order
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
  return ss;
}
__device__ __forceinline__ float fexp(float x) { return __builtin_amdgcn_exp2f(x * KDN_LOG2E); }
// 2^x on the hardware exp2 (one v_exp_f32): results below 2^-126 flush towards zero, where exp2f
// would produce denormals; every use multiplies it with O(1) terms, so the difference is below 1e-38.
__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fsoftplus_y(float x, float y, float d) {  // y = e^min(x, 20), d = 1 + y
  // every operand is computed first, so both conditionals are selects (a conditional over an
  // expression is emitted as a branch, and the logarithm would be sunk into it)
  const float l = __builtin_amdgcn_logf(d) * KDN_LN2;
  const float small = y * (1.f - 0.5f * y);
  const float t = y < 1e-3f ? small : l;
  return x > 20.f ? x : t;
}
__device__ __forceinline__ float fsoftplus(float x) {
  const float y = fexp(x > 20.f ? 20.f : x);
  return fsoftplus_y(x, y, 1.f + y);
}
__device__ __forceinline__ void fsoftplus_sigmoid(float x, float& sp, float& sg) {
  const float y = fexp(x > 20.f ? 20.f : x);
  const float d = 1.f + y;
  sg = y * frcp(d);
  sp = fsoftplus_y(x, y, d);
}
// sigmoid(x) = 1 / (1 + e^-x) on the hardware exp and reciprocal
__device__ __forceinline__ float fsigmoid(float x) { return frcp(1.f + fexp(-x)); }

// ---- wave64 reductions -----------------------------------------------------------
// x + (x of lane ^ 1 or ^ 2) by a DPP quad permutation, or + (x of lane 7 - i in its 8-lane group /
// 15 - i in its 16-lane row) by a DPP mirror, or + (x of lane ^ 16) by a swizzle: one instruction each,
// no lane-index arithmetic and no LDS-crossbar round trip.  Every lane of the group must be active.
// Used as the steps of an xor butterfly (x += x[lane ^ o], o = 1, 2, 4, 8, 16) they add the same values:
// after the two quad steps all lanes of a quad hold the same sum, so the half-row mirror adds the same
// partner as lane ^ 4 would, and after it the row mirror the same as lane ^ 8; the result is
// bit-identical to the butterfly's.
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror
constexpr int kDppMirror = 0x140;      // row_mirror
template <int CTRL>
__device__ __forceinline__ float dpp_add(float x) {
  return x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float swz16_add(float x) {
  return x + __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x401F));  // and 31, xor 16
}
// the xor butterfly over the 16 lanes of a row (o = 1, 2, 4, 8), bit-identical to it
__device__ __forceinline__ float row16_sum(float x) {
  return dpp_add<kDppMirror>(dpp_add<kDppHalfMirror>(dpp_add<kDppXor2>(dpp_add<kDppXor1>(x))));
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Block-wide sum for blockDim.x <= 1024; `scratch` holds >= 16 floats. Result valid in all threads.
__device__ __forceinline__ float block_sum(float v, float* scratch) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) scratch[w] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; ++i) t += scratch[i];
  return t;
}

namespace {
// out[j] = sum_p part[p * stride + j] for j < n, deterministic order: block = 64 outputs x 4
// partial stripes (each 8-way unrolled over p), stripes combined in order.  grid (ceil(n/64), S): with
// S > 1 segment y sums rows [NP y / S, NP (y + 1) / S) into out[y * n + j] (a second call with NP = S
// finishes), so a tall partial array is reduced by S times more workgroups.
__global__ __launch_bounds__(256) void reduce_partials_vec_kernel(const float* __restrict__ part, int NP,
                                                                  int64_t stride, int n, float* __restrict__ out) {
  __shared__ float s[4][64];
  const int jj = threadIdx.x & 63, st4 = threadIdx.x >> 6, j = blockIdx.x * 64 + jj;
  const int p0 = (int)((int64_t)NP * blockIdx.y / gridDim.y), p1 = (int)((int64_t)NP * (blockIdx.y + 1) / gridDim.y);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (j < n) {
    int pp = p0 + st4;
    for (; pp + 28 < p1; pp += 32) {
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[q] += part[(int64_t)(pp + 4 * q) * stride + j];
    }
    for (; pp < p1; pp += 4) acc[0] += part[(int64_t)pp * stride + j];
  }
  s[st4][jj] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  __syncthreads();
  if (st4 == 0 && j < n) out[(int64_t)blockIdx.y * n + j] = (s[0][jj] + s[1][jj]) + (s[2][jj] + s[3][jj]);
}

// Several partial reductions (each as reduce_partials_vec_kernel, same summation order) and the
// prior-precision VJP in one launch: workgroup x serves the reduction whose block range holds it (64
// outputs per workgroup); the workgroups past the last one form the VJP.  grid (blocks, S): as in
// reduce_partials_vec_kernel, row segment y sums rows [NP y / S, NP (y + 1) / S) into out[y * n + j] (the
// VJP runs in segment 0).  The launches this replaces were each a few microseconds of dispatch.
struct PartSeg {
  const float* part;
  int64_t stride;
  int n;
  float* out;
};
struct PartSegs {
  PartSeg seg[4];
  int nseg;
  // The prior precision's cotangent over H entries: d = dmu (null: 0) plus, with rows_to_param,
  // rows = sum over b < nrows of dmu_rows[b * H + h] (per batch row values, summed in order of b).
  // dmu_param = d * sigmoid(mu_param) when dmu_param != null; dmu_sum = rows when dmu_sum != null.
  const float* mu_param;
  const float* dmu;
  const float* dmu_rows;
  int nrows, rows_to_param;
  int H;
  float* dmu_param;
  float* dmu_sum;
};
inline int part_segs_blocks(const PartSegs& P) {
  int nb = 0;
  for (int i = 0; i < P.nseg; ++i) nb += (P.seg[i].n + 63) / 64;
  return nb + ((P.dmu_param || P.dmu_sum) ? (P.H + 255) / 256 : 0);
}
__global__ __launch_bounds__(256) void reduce_partials_multi_kernel(PartSegs P, int NP) {
  __shared__ float s[4][64];
  int blk = blockIdx.x, i = 0;
  for (; i < P.nseg; ++i) {
    const int nb = (P.seg[i].n + 63) / 64;
    if (blk < nb) break;
    blk -= nb;
  }
  if (i == P.nseg) {  // the prior-precision VJP
    if (blockIdx.y != 0) return;
    const int hh = blk * 256 + threadIdx.x;
    if (hh < P.H) {
      float rows = 0.f;
      for (int bb = 0; bb < P.nrows; ++bb) rows += P.dmu_rows[(int64_t)bb * P.H + hh];
      const float d = (P.dmu ? P.dmu[hh] : 0.f) + (P.rows_to_param ? rows : 0.f);
      if (P.dmu_param) P.dmu_param[hh] = d * sigmoidf(P.mu_param[hh]);
      if (P.dmu_sum) P.dmu_sum[hh] = rows;
    }
    return;
  }
  const PartSeg g = P.seg[i];
  const int jj = threadIdx.x & 63, st4 = threadIdx.x >> 6, j = blk * 64 + jj;
  const int p0 = (int)((int64_t)NP * blockIdx.y / gridDim.y), p1 = (int)((int64_t)NP * (blockIdx.y + 1) / gridDim.y);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (j < g.n) {
    int pp = p0 + st4;
    for (; pp + 28 < p1; pp += 32) {
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[q] += g.part[(int64_t)(pp + 4 * q) * g.stride + j];
    }
    for (; pp < p1; pp += 4) acc[0] += g.part[(int64_t)pp * g.stride + j];
  }
  s[st4][jj] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  __syncthreads();
  if (st4 == 0 && j < g.n) g.out[(int64_t)blockIdx.y * g.n + j] = (s[0][jj] + s[1][jj]) + (s[2][jj] + s[3][jj]);
}
}  // namespace

// Error codes returned by the C ABI besides hipError_t values (KDN_ERR_ARG) come from the public header.
#define KDN_CHECK_LAUNCH()                       \
  do {                                           \
    hipError_t e_ = hipGetLastError();           \
    if (e_ != hipSuccess) return (int)e_;        \
  } while (0)
