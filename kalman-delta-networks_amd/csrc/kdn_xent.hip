// Fused cross-entropy over a logits matrix [n_rows, n_cols] (the language-model loss): per row the
// log-sum-exp of the scaled logits, the loss with optional label smoothing and z-loss, and the
// gradient with respect to the logits.  Semantics of lit_gpt/fused_cross_entropy.py:29-150
// (forward :29-100, backward :103-150), including its vocabulary-split mode, in which each of
// several ranks holds n_cols of total_classes classes from class_start_idx on.
//
// Both passes are HBM-bound: the forward reads every logit once (one workgroup per row, an
// online log-sum-exp in the base-2 domain, one exponential per logit plus one per 8-vector
// group), the backward reads every logit and writes its gradient once (several workgroups per
// row).  Rows are read in 16-byte vectors when the rows are 16-byte aligned.
#include "kdn_common.h"

namespace {

constexpr int kXentThreads = 256;
constexpr int kXentBwdVectors = 4;  // backward: 16-byte vectors in flight per thread

template <typename T> __device__ __forceinline__ float to_f(T x);
template <> __device__ __forceinline__ float to_f<float>(float x) { return x; }
template <> __device__ __forceinline__ float to_f<bf16_t>(bf16_t x) { return bf2f(x); }
template <> __device__ __forceinline__ float to_f<_Float16>(_Float16 x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f(float x);
template <> __device__ __forceinline__ float from_f<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16_t from_f<bf16_t>(float x) { return f2bf(x); }
template <> __device__ __forceinline__ _Float16 from_f<_Float16>(float x) { return (_Float16)x; }

// VEC consecutive elements from p (16 bytes when VEC > 1; p then 16-byte aligned)
template <typename T, int VEC> __device__ __forceinline__ void ldv(const T* p, float (&f)[VEC]) {
  if constexpr (VEC == 1) {
    f[0] = to_f<T>(p[0]);
  } else {
    static_assert(VEC * sizeof(T) == 16, "16-byte vectors");
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const T* e = reinterpret_cast<const T*>(&u);
#pragma unroll
    for (int i = 0; i < VEC; ++i) f[i] = to_f<T>(e[i]);
  }
}
template <typename T, int VEC> __device__ __forceinline__ void stv(T* p, const float (&f)[VEC]) {
  if constexpr (VEC == 1) {
    p[0] = from_f<T>(f[0]);
  } else {
    uint4 u;
    T* e = reinterpret_cast<T*>(&u);
#pragma unroll
    for (int i = 0; i < VEC; ++i) e[i] = from_f<T>(f[i]);
    *reinterpret_cast<uint4*>(p) = u;
  }
}

// The same through a buffer resource over the row (wave-uniform base): a load past the
// resource's size returns 0 and a store there is dropped, so guarded accesses need no branch
// and a thread's loads are all issued before the first wait.  byte_off is VEC-element aligned.
template <typename T, int VEC> __device__ __forceinline__ void ldv_buf(bufrsrc r, uint32_t byte_off, float (&f)[VEC]) {
  if constexpr (VEC == 1) {
    if constexpr (sizeof(T) == 4) {
      f[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 0));
    } else {
      const uint16_t u = __builtin_amdgcn_raw_buffer_load_b16(r, byte_off, 0, 0);
      f[0] = to_f<T>(__builtin_bit_cast(T, u));
    }
  } else {
    const u32x4 u = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
    const T* e = reinterpret_cast<const T*>(&u);
#pragma unroll
    for (int i = 0; i < VEC; ++i) f[i] = to_f<T>(e[i]);
  }
}
template <typename T, int VEC> __device__ __forceinline__ void stv_buf(bufrsrc r, uint32_t byte_off, const float (&f)[VEC]) {
  if constexpr (VEC == 1) {
    if constexpr (sizeof(T) == 4) {
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(f[0]), r, byte_off, 0, 0);
    } else {
      __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, from_f<T>(f[0])), r, byte_off, 0, 0);
    }
  } else {
    u32x4 u;
    T* e = reinterpret_cast<T*>(&u);
#pragma unroll
    for (int i = 0; i < VEC; ++i) e[i] = from_f<T>(f[i]);
    __builtin_amdgcn_raw_buffer_store_b128(u, r, byte_off, 0, 0);
  }
}

__device__ __forceinline__ int64_t load_label(const void* labels, int i64, int row) {
  return i64 ? reinterpret_cast<const int64_t*>(labels)[row] : (int64_t)reinterpret_cast<const int32_t*>(labels)[row];
}

// (m, l) with l = sum 2^(y - m): merge b into a.  m = -inf means an empty sum (l = 0).
__device__ __forceinline__ void lse_merge(float& m, float& l, float mb, float lb) {
  const float mn = fmaxf(m, mb);
  if (mn == -INFINITY) return;
  l = l * __builtin_amdgcn_exp2f(m - mn) + lb * __builtin_amdgcn_exp2f(mb - mn);
  m = mn;
}

// Forward: one workgroup per row.  In the base-2 domain y = logit * logit_scale * log2(e); per
// thread a running (m, l) over its vectors, merged across the wave with shuffles and across waves
// through LDS.  logit_scale > 0, so a vector group's maximum is taken on the raw logits and each
// logit then costs one fma and one v_exp_f32 (terms below 2^-126 of the maximum flush to 0).
template <typename T, int VEC, bool SMOOTH>
__global__ __launch_bounds__(kXentThreads) void xent_fwd_kernel(
    const T* __restrict__ logits, int64_t ls, const void* __restrict__ labels, int labels_i64, int n_cols,
    float smoothing, float logit_scale, float lse_square_scale, int64_t ignore_index, int64_t total_classes,
    int64_t class_start, int split, int pre_lse, float* __restrict__ losses, float* __restrict__ lse_io,
    float* __restrict__ z_losses) {
  constexpr int U = 4;  // vectors in flight per thread
  const int row = blockIdx.x, t = threadIdx.x;
  const T* x = logits + (int64_t)row * ls;
  const float ys = logit_scale * KDN_LOG2E;
  float m = -INFINITY, l = 0.f, sx = 0.f;
  if (!pre_lse) {
    const int nvec = n_cols / VEC;
    const bufrsrc rx = make_buf(x, (uint32_t)nvec * VEC * sizeof(T));  // the row's whole vectors
    for (int v0 = t; v0 < nvec; v0 += kXentThreads * U) {
      float e[U][VEC];
#pragma unroll
      for (int u = 0; u < U; ++u) ldv_buf<T, VEC>(rx, (uint32_t)(v0 + kXentThreads * u) * (VEC * sizeof(T)), e[u]);
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (v0 + kXentThreads * u >= nvec) {
#pragma unroll
          for (int i = 0; i < VEC; ++i) e[u][i] = -INFINITY;
        }
      float cm = -INFINITY, cs = 0.f;
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          cm = fmaxf(cm, e[u][i]);
          if (SMOOTH && v0 + kXentThreads * u < nvec) cs += e[u][i];
        }
      if (SMOOTH) sx += cs * logit_scale;
      if (cm == -INFINITY) continue;
      const float mn = fmaxf(m, cm * ys);
      float s = 0.f;
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int i = 0; i < VEC; ++i) s += __builtin_amdgcn_exp2f(fmaf(e[u][i], ys, -mn));
      l = l * __builtin_amdgcn_exp2f(m - mn) + s;
      m = mn;
    }
    for (int c = nvec * VEC + t; c < n_cols; c += kXentThreads) {  // tail columns
      const float raw = to_f<T>(x[c]);
      if (SMOOTH) sx += raw * logit_scale;
      lse_merge(m, l, raw * ys, 1.f);
    }
    // wave merge
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float mo = __shfl_xor(m, o, 64), lo = __shfl_xor(l, o, 64);
      lse_merge(m, l, mo, lo);
      if (SMOOTH) sx += __shfl_xor(sx, o, 64);
    }
    __shared__ float sm[kXentThreads / 64], sl[kXentThreads / 64], ss[kXentThreads / 64];
    const int w = t / 64;
    if ((t & 63) == 0) sm[w] = m, sl[w] = l, ss[w] = sx;
    __syncthreads();
    if (t != 0) return;
    m = sm[0], l = sl[0], sx = ss[0];
#pragma unroll
    for (int i = 1; i < kXentThreads / 64; ++i) {
      lse_merge(m, l, sm[i], sl[i]);
      sx += ss[i];
    }
  } else if (t != 0) {
    return;
  }
  // thread 0: the row's loss
  float lse;
  if (pre_lse) {
    lse = lse_io[row];
  } else {
    lse = (m + log2f(l)) * KDN_LN2;  // m = -inf (all logits -inf) gives -inf, as log(0) does
    lse_io[row] = lse;
  }
  const int64_t label = load_label(labels, labels_i64, row);
  float loss = 0.f, z = 0.f;
  if (label != ignore_index) {
    const float lse_part = split ? 0.f : lse;
    const int64_t li = label - class_start;
    if (li >= 0 && li < n_cols) {
      const float xl = to_f<T>(x[li]) * logit_scale;
      loss = SMOOTH ? lse_part - smoothing * sx / (float)total_classes - (1.f - smoothing) * xl : lse_part - xl;
    } else {
      // the label is another rank's class (split) or out of range: only the smoothing term
      loss = SMOOTH ? smoothing * (lse_part - sx / (float)total_classes) : 0.f;
    }
    if (!split) {
      z = lse_square_scale * lse * lse;
      loss += z;
    }
  }
  losses[row] = loss;
  if (!split && z_losses) z_losses[row] = z;
}

template <typename T, int VEC>
void launch_fwd(const void* logits, int64_t ls, const void* labels, int labels_i64, int n_rows, int n_cols,
                float smoothing, float logit_scale, float lse_sq, int64_t ignore_index, int64_t total, int64_t start,
                int split, int pre_lse, float* losses, float* lse, float* z, hipStream_t stream) {
  const dim3 grid(n_rows), block(kXentThreads);
  if (smoothing > 0.f)
    hipLaunchKernelGGL((xent_fwd_kernel<T, VEC, true>), grid, block, 0, stream, (const T*)logits, ls, labels,
                       labels_i64, n_cols, smoothing, logit_scale, lse_sq, ignore_index, total, start, split, pre_lse,
                       losses, lse, z);
  else
    hipLaunchKernelGGL((xent_fwd_kernel<T, VEC, false>), grid, block, 0, stream, (const T*)logits, ls, labels,
                       labels_i64, n_cols, smoothing, logit_scale, lse_sq, ignore_index, total, start, split, pre_lse,
                       losses, lse, z);
}

// Backward: workgroup b covers columns [cb * kXentThreads * VEC * U, ...) of row b / ncb.
// dlogit = dloss * logit_scale * (p (1 + 2 z lse) - [c == label](1 - s) - s / total),
// p = exp(scale * logit - lse), dloss = 0 on ignored rows: per element one fma for the exponent,
// one v_exp_f32 and one fma; the label's column is corrected in the one vector that holds it.
// dlogits may alias logits (each element is read and then written by the same thread).
template <typename T, int VEC>
__global__ __launch_bounds__(kXentThreads) void xent_bwd_kernel(
    T* dlogits, int64_t dls, const float* __restrict__ dlosses, int64_t dlosses_stride, const T* logits, int64_t ls,
    const float* __restrict__ lse_in, const void* __restrict__ labels, int labels_i64, int n_cols, int ncb,
    float smoothing, float logit_scale, float lse_square_scale, int64_t ignore_index, int64_t total_classes,
    int64_t class_start) {
  constexpr int U = kXentBwdVectors;
  const int row = blockIdx.x / ncb, cb = blockIdx.x % ncb;
  const int64_t label = load_label(labels, labels_i64, row);
  const float dloss = label != ignore_index ? dlosses[(int64_t)row * dlosses_stride] : 0.f;
  const float lse = lse_in[row];
  const float g = dloss * logit_scale;
  const float gp = g * (1.f + 2.f * lse_square_scale * lse);  // multiplies p
  const float gneg = g * (smoothing / (float)total_classes);  // subtracted everywhere
  const float gpos = g * (1.f - smoothing);                   // subtracted at the label
  const float ys = logit_scale * KDN_LOG2E, lse2 = lse * KDN_LOG2E;
  const int64_t li = label - class_start;  // a column of this row's slice when 0 <= li < n_cols
  const T* x = logits + (int64_t)row * ls;
  T* dx = dlogits + (int64_t)row * dls;
  const int nvec = n_cols / VEC;
  const uint32_t vbytes = (uint32_t)nvec * VEC * sizeof(T);  // the row's whole vectors
  const bufrsrc rx = make_buf(x, vbytes), rdx = make_buf(dx, vbytes);
  const int v0 = cb * kXentThreads * U + threadIdx.x;
  float e[U][VEC];
#pragma unroll
  for (int u = 0; u < U; ++u) ldv_buf<T, VEC>(rx, (uint32_t)(v0 + kXentThreads * u) * (VEC * sizeof(T)), e[u]);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int v = v0 + kXentThreads * u;
#pragma unroll
    for (int i = 0; i < VEC; ++i) e[u][i] = fmaf(gp, __builtin_amdgcn_exp2f(fmaf(e[u][i], ys, -lse2)), -gneg);
    const int64_t off = li - (int64_t)v * VEC;
    if (off >= 0 && off < VEC) {
#pragma unroll
      for (int i = 0; i < VEC; ++i)
        if (i == off) e[u][i] -= gpos;
    }
    stv_buf<T, VEC>(rdx, (uint32_t)v * (VEC * sizeof(T)), e[u]);  // dropped past the row's vectors
  }
  if (cb == ncb - 1) {  // tail columns, by the row's last workgroup
    for (int c = nvec * VEC + threadIdx.x; c < n_cols; c += kXentThreads) {
      float d = fmaf(gp, __builtin_amdgcn_exp2f(fmaf(to_f<T>(x[c]), ys, -lse2)), -gneg);
      if (c == li) d -= gpos;
      dx[c] = from_f<T>(d);
    }
  }
}

template <typename T, int VEC>
int launch_bwd(void* dlogits, int64_t dls, const float* dlosses, int64_t dstride, const void* logits, int64_t ls,
               const float* lse, const void* labels, int labels_i64, int n_rows, int n_cols, float smoothing,
               float logit_scale, float lse_sq, int64_t ignore_index, int64_t total, int64_t start,
               hipStream_t stream) {
  const int per = kXentThreads * kXentBwdVectors;  // vectors per workgroup
  const int nvec = n_cols / VEC;
  const int ncb = nvec > 0 ? (nvec + per - 1) / per : 1;  // the last block also takes the tail columns
  if ((int64_t)n_rows * ncb > INT32_MAX) return KDN_ERR_ARG;
  hipLaunchKernelGGL((xent_bwd_kernel<T, VEC>), dim3(n_rows * ncb), dim3(kXentThreads), 0, stream, (T*)dlogits, dls,
                     dlosses, dstride, (const T*)logits, ls, lse, labels, labels_i64, n_cols, ncb, smoothing,
                     logit_scale, lse_sq, ignore_index, total, start);
  return 0;
}

// 16-byte vectors when the base and every row start are 16-byte aligned
bool vec_ok(const void* p, int64_t row_stride, int esize) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0 && (row_stride * esize) % 16 == 0;
}

// rows are addressed through buffer resources with 32-bit byte offsets: at most 2^30 bytes a row
bool args_ok(int dtype, int n_rows, int n_cols, int64_t total_classes, int64_t class_start, float logit_scale) {
  return dtype >= 0 && dtype <= 2 && n_rows >= 0 && n_cols > 0 && (int64_t)n_cols * (dtype == 0 ? 4 : 2) <= (1 << 30) &&
         total_classes >= n_cols && class_start >= 0 && class_start + n_cols <= total_classes && logit_scale > 0.f;
}

}  // namespace

extern "C" int kdn_xent_fwd(const void* logits, int logits_dtype, int64_t logits_row_stride, const void* labels,
                            int labels_i64, int n_rows, int n_cols, float smoothing, float logit_scale,
                            float lse_square_scale, int64_t ignore_index, int64_t total_classes,
                            int64_t class_start_idx, int split, int precomputed_lse, float* losses, float* lse,
                            float* z_losses, hipStream_t stream) {
  if (!args_ok(logits_dtype, n_rows, n_cols, total_classes, class_start_idx, logit_scale)) return KDN_ERR_ARG;
  if (logits_row_stride < n_cols || !(smoothing >= 0.f && smoothing <= 1.f)) return KDN_ERR_ARG;
  if (precomputed_lse && (smoothing != 0.f || logit_scale != 1.f)) return KDN_ERR_ARG;
  if (n_rows == 0) return 0;
  if (!logits || !labels || !losses || !lse || (!split && !z_losses)) return KDN_ERR_ARG;
  const int64_t ls = logits_row_stride;
#define KDN_XENT_FWD(T, VEC)                                                                                          \
  launch_fwd<T, VEC>(logits, ls, labels, labels_i64, n_rows, n_cols, smoothing, logit_scale, lse_square_scale,      \
                     ignore_index, total_classes, class_start_idx, split, precomputed_lse, losses, lse, z_losses,    \
                     stream)
  if (logits_dtype == 0) {
    if (vec_ok(logits, ls, 4)) KDN_XENT_FWD(float, 4);
    else KDN_XENT_FWD(float, 1);
  } else if (logits_dtype == 1) {
    if (vec_ok(logits, ls, 2)) KDN_XENT_FWD(bf16_t, 8);
    else KDN_XENT_FWD(bf16_t, 1);
  } else {
    if (vec_ok(logits, ls, 2)) KDN_XENT_FWD(_Float16, 8);
    else KDN_XENT_FWD(_Float16, 1);
  }
#undef KDN_XENT_FWD
  KDN_CHECK_LAUNCH();
  return 0;
}

extern "C" int kdn_xent_bwd(void* dlogits, int64_t dlogits_row_stride, const float* dlosses, int64_t dlosses_stride,
                            const void* logits, int logits_dtype, int64_t logits_row_stride, const float* lse,
                            const void* labels, int labels_i64, int n_rows, int n_cols, float smoothing,
                            float logit_scale, float lse_square_scale, int64_t ignore_index, int64_t total_classes,
                            int64_t class_start_idx, hipStream_t stream) {
  if (!args_ok(logits_dtype, n_rows, n_cols, total_classes, class_start_idx, logit_scale)) return KDN_ERR_ARG;
  if (logits_row_stride < n_cols || dlogits_row_stride < n_cols || !(smoothing >= 0.f && smoothing <= 1.f))
    return KDN_ERR_ARG;
  if (n_rows == 0) return 0;
  if (!dlogits || !dlosses || !logits || !lse || !labels) return KDN_ERR_ARG;
  // in place only row for row
  if (dlogits == logits && dlogits_row_stride != logits_row_stride) return KDN_ERR_ARG;
  const int64_t ls = logits_row_stride, dls = dlogits_row_stride;
  int rc;
#define KDN_XENT_BWD(T, VEC)                                                                                          \
  rc = launch_bwd<T, VEC>(dlogits, dls, dlosses, dlosses_stride, logits, ls, lse, labels, labels_i64, n_rows, n_cols, \
                          smoothing, logit_scale, lse_square_scale, ignore_index, total_classes, class_start_idx,     \
                          stream)
  const int es = logits_dtype == 0 ? 4 : 2;
  const bool vec = vec_ok(logits, ls, es) && vec_ok(dlogits, dls, es);
  if (logits_dtype == 0) {
    if (vec) KDN_XENT_BWD(float, 4);
    else KDN_XENT_BWD(float, 1);
  } else if (logits_dtype == 1) {
    if (vec) KDN_XENT_BWD(bf16_t, 8);
    else KDN_XENT_BWD(bf16_t, 1);
  } else {
    if (vec) KDN_XENT_BWD(_Float16, 8);
    else KDN_XENT_BWD(_Float16, 1);
  }
#undef KDN_XENT_BWD
  if (rc) return rc;
  KDN_CHECK_LAUNCH();
  return 0;
}
