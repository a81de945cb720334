// Elementwise frontends of the KDN scan: iso gate, diag retention/noise frontend,
// q/k row normalisations.  HBM-bound; one workgroup per (batch, chunk, head) tile.
//
// Reference behaviour restated (ngocbh/kalman-delta-networks):
//   iso gate      lit_gpt/kdn_ops/iso_kdn_chunk.py:739-1009
//   diag frontend lit_gpt/kdn_ops/diag_kdn_chunk.py:1866-2016
//   diag norm     lit_gpt/kdn_ops/diag_kdn_chunk.py:193-353
//   FLA l2norm    iso_kdn_chunk.py:2203-2204,2229-2230 (x * rsqrt(sum x^2 + eps))
#include "kdn_common.h"
#include "kdn_iso_gain.h"
#include "../../include/kdn.h"

namespace {

constexpr int kMaxChunk = 64;

// ---------------------------------------------------------------------------
// iso gate forward.  grid (H * B * NT) with the head fastest, block 256 (thread = key channel).
// ---------------------------------------------------------------------------
template <typename TG, typename TO>
__global__ __launch_bounds__(256) void iso_gate_fwd_kernel(
    const TG* __restrict__ g_raw, const TO* __restrict__ orr, int64_t orr_sb, int64_t orr_st,
    const float* __restrict__ omega_bias, const float* __restrict__ r_bias, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, const float* __restrict__ mu_param, float omega_min, float r_min,
    int T, int H, int K, int chunk, int NT, float* __restrict__ g_cumsum, float* __restrict__ a_out,
    float* __restrict__ omega_out, float* __restrict__ r_out, float* __restrict__ mu_out) {
  __shared__ float s_e2[kMaxChunk][257];
  const int h = blockIdx.x % H, b = blockIdx.x / H / NT, nt = blockIdx.x / H % NT, i = threadIdx.x;
  const int t0 = nt * chunk, L = min(chunk, T - t0);
  const float rate = __expf(A_log[h]);
  if (i < K) {
    const float bias = dt_bias[h * K + i];
    float acc = 0.f;
    for (int t = 0; t < L; ++t) {
      const int64_t off = (((int64_t)b * T + t0 + t) * H + h) * K + i;
      const float g = -rate * softplusf(ld(g_raw, off) + bias);
      acc += g;
      g_cumsum[off] = acc * KDN_LOG2E;
      s_e2[t][i] = __expf(2.f * g);
    }
  }
  __syncthreads();
  if (i < L) {
    float s = 0.f;
    for (int j = 0; j < K; ++j) s += s_e2[i][j];
    const int64_t o = ((int64_t)b * T + t0 + i) * H + h;
    a_out[o] = s / (float)K;
    const int64_t ro = (int64_t)b * orr_sb + (int64_t)(t0 + i) * orr_st + h;
    omega_out[o] = omega_min + softplusf(ld(orr, ro) + omega_bias[h]);
    r_out[o] = r_min + softplusf(ld(orr, ro + H) + r_bias[h]);
  }
  if (blockIdx.x < H && i == 0) mu_out[h] = 0.1f + softplusf(mu_param[h]);
}

// iso gate backward.  Writes per-tile partial sums; reduce_partials_multi_kernel finishes them.
template <typename TG, typename TO>
__global__ __launch_bounds__(256) void iso_gate_bwd_kernel(
    const TG* __restrict__ g_raw, const TO* __restrict__ orr, int64_t orr_sb, int64_t orr_st,
    const float* __restrict__ omega_bias, const float* __restrict__ r_bias, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, const float* __restrict__ dg_pre, const float* __restrict__ da,
    const float* __restrict__ domega, const float* __restrict__ dr, int T, int H, int K, int chunk, int NT,
    TG* __restrict__ dg_raw, TO* __restrict__ dorr, float* __restrict__ part_A, float* __restrict__ part_dt,
    float* __restrict__ part_bias) {
  __shared__ float red[16];
  const int h = blockIdx.x % H, b = blockIdx.x / H / NT, nt = blockIdx.x / H % NT, i = threadIdx.x;
  const int t0 = nt * chunk, L = min(chunk, T - t0);
  const int p = blockIdx.x / H;  // partial index (b, nt)
  const float rate = __expf(A_log[h]);
  float dA_term = 0.f;
  if (i < K) {
    const float bias = dt_bias[h * K + i];
    float acc = 0.f, ddt = 0.f;
    for (int t = L - 1; t >= 0; --t) {
      const int64_t off = (((int64_t)b * T + t0 + t) * H + h) * K + i;
      const float x = ld(g_raw, off) + bias;
      const float g = -rate * softplusf(x);
      float dgl = 0.f;
      if (dg_pre) { acc += dg_pre[off]; dgl = acc; }
      if (da) dgl += da[((int64_t)b * T + t0 + t) * H + h] * (2.f / (float)K) * __expf(2.f * g);
      const float dgr = dgl * (-rate) * sigmoidf(x);
      if (dg_raw) st(dg_raw, off, dgr);
      dA_term += dgl * g;
      ddt += dgr;
    }
    if (part_dt) part_dt[((int64_t)p * H + h) * K + i] = ddt;
  }
  float dob = 0.f, drb = 0.f;
  if (i < L) {
    const int64_t o = ((int64_t)b * T + t0 + i) * H + h;
    const int64_t ro = (int64_t)b * orr_sb + (int64_t)(t0 + i) * orr_st + h;
    if (domega) dob = domega[o] * sigmoidf(ld(orr, ro) + omega_bias[h]);
    if (dr) drb = dr[o] * sigmoidf(ld(orr, ro + H) + r_bias[h]);
    if (dorr) {
      const int64_t wo = ((int64_t)b * T + t0 + i) * (2 * H) + h;
      st(dorr, wo, dob);
      st(dorr, wo + H, drb);
    }
  }
  const float sA = block_sum(dA_term, red);
  if (part_A && i == 0) part_A[(int64_t)p * H + h] = sA;
  const float sO = block_sum(dob, red);
  const float sR = block_sum(drb, red);
  if (part_bias && i == 0) {
    part_bias[(int64_t)p * 2 * H + h] = sO;
    part_bias[(int64_t)p * 2 * H + H + h] = sR;
  }
}

// ---------------------------------------------------------------------------
// Vectorised iso gate (K % 8 == 0): thread = 8 consecutive channels x TPG tokens of the chunk.
// tid = tg * CG + cg (CG = K/8 channel groups, TG = 256/CG token groups).  The chunk-local
// prefix (forward) / suffix (backward) over token groups goes through LDS group totals.
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void load8(const T* p, float* f);
template <>
__device__ __forceinline__ void load8<bf16_t>(const bf16_t* p, float* f) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    f[2 * q] = __uint_as_float(w[q] << 16);
    f[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
  }
}
template <>
__device__ __forceinline__ void load8<float>(const float* p, float* f) {
  const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
  f[0] = a.x, f[1] = a.y, f[2] = a.z, f[3] = a.w, f[4] = b.x, f[5] = b.y, f[6] = b.z, f[7] = b.w;
}
template <typename T>
__device__ __forceinline__ void store8(T* p, const float* f);
template <>
__device__ __forceinline__ void store8<bf16_t>(bf16_t* p, const float* f) {
  uint32_t w[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) w[q] = (uint32_t)f2bf(f[2 * q]) | ((uint32_t)f2bf(f[2 * q + 1]) << 16);
  *reinterpret_cast<uint4*>(p) = uint4{w[0], w[1], w[2], w[3]};
}
template <>
__device__ __forceinline__ void store8<float>(float* p, const float* f) {
  reinterpret_cast<float4*>(p)[0] = float4{f[0], f[1], f[2], f[3]};
  reinterpret_cast<float4*>(p)[1] = float4{f[4], f[5], f[6], f[7]};
}

// s_tot [TGN][K] holds each token group's per-channel totals; replace them in place by the exclusive
// prefix over the groups (forward: the earlier groups' sum, taken in group order, as a left fold from 0) or
// suffix (backward: the later groups' sum, accumulated from the last group down).  One thread per channel
// walks the groups, so the reads and writes are consecutive words; the caller's barriers order the
// writes of the totals before this and the reads of the prefixes after.
__device__ __forceinline__ void group_prefix_excl(float* s_tot, int K, int TGN, int tid) {
  if (tid < K) {
    float run = 0.f;
#pragma unroll 8
    for (int q = 0; q < TGN; ++q) {
      const float x = s_tot[q * K + tid];
      s_tot[q * K + tid] = run;
      run += x;
    }
  }
  __syncthreads();
}
__device__ __forceinline__ void group_suffix_excl(float* s_tot, int K, int TGN, int tid) {
  if (tid < K) {
    float run = 0.f;
#pragma unroll 8
    for (int q = TGN - 1; q >= 0; --q) {
      const float x = s_tot[q * K + tid];
      s_tot[q * K + tid] = run;
      run += x;
    }
  }
  __syncthreads();
}

// grid (H * B * NT) with the head fastest, block 256.  With MAPS (chunk = 64, the fused front) the
// workgroup also writes its chunk's gain map gain_maps[(b * H + h) * NT + nt] (posterior scale gain_s)
// from the a, omega, r it has just produced.
template <typename TG, typename TO, bool MAPS>
__global__ __launch_bounds__(256) void iso_gate_fwd_vec_kernel(
    const TG* __restrict__ g_raw, const TO* __restrict__ orr, int64_t orr_sb, int64_t orr_st,
    const float* __restrict__ omega_bias, const float* __restrict__ r_bias, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, const float* __restrict__ mu_param, float omega_min, float r_min,
    int T, int H, int K, int chunk, int NT, float* __restrict__ g_cumsum, float* __restrict__ a_out,
    float* __restrict__ omega_out, float* __restrict__ r_out, float* __restrict__ mu_out,
    float4* __restrict__ gain_maps, float gain_s) {
  __shared__ __attribute__((aligned(16))) float s_tot[256 * 8];  // [tg][K] group totals (TG * K = 2048)
  __shared__ float s_ga[MAPS ? kIsoChunk : 1];  // MAPS: a of each token
  const int CG = K / 8, TGN = 256 / CG, TPG = (chunk + TGN - 1) / TGN;
  const int h = blockIdx.x % H, b = blockIdx.x / H / NT, nt = blockIdx.x / H % NT, tid = threadIdx.x;
  const int cg = tid % CG, tg = tid / CG, i0 = 8 * cg;
  const int t0 = nt * chunk, L = min(chunk, T - t0);
  const float rate = __expf(A_log[h]);  // once per thread
  float bias[8];
  load8<float>(dt_bias + h * K + i0, bias);
  // per-token omega / r: thread tid owns token tid (chunk <= 256; loads clamped to the chunk)
  const int64_t sro = (int64_t)b * orr_sb + (int64_t)(t0 + min(tid, L - 1)) * orr_st + h;
  const float or_t = ld(orr, sro), rr_t = ld(orr, sro + H);
  // every load of this thread's tokens goes out first (rows clamped to the chunk; the clamped
  // duplicates are never used), so the thread waits for memory once
  float xr[4][8];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int t = min(tg * TPG + u, L - 1);
    load8<TG>(g_raw + (((int64_t)b * T + t0 + t) * H + h) * K + i0, xr[u]);
  }
  const float om_t = omega_min + fsoftplus(or_t + omega_bias[h]), r_t = r_min + fsoftplus(rr_t + r_bias[h]);
  if (tid < L) {
    const int64_t o = ((int64_t)b * T + t0 + tid) * H + h;
    omega_out[o] = om_t;
    r_out[o] = r_t;
  }
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const float c2g = -2.f * rate * KDN_LOG2E;  // e^{2 g} for g = -rate sp is 2^{c2g sp}
  float pre[4][8];  // local inclusive prefix per token (TPG <= 4 when K >= 64 and chunk <= 64)
  float e2[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int t = tg * TPG + u;
    e2[u] = 0.f;
    if (u < TPG && t < L) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float sp = fsoftplus(xr[u][j] + bias[j]);
        const float g = -rate * sp;
        acc[j] += g;
        pre[u][j] = acc[j];
        e2[u] += fexp2(sp * c2g);  // e^{2 g} = 2^{(-2 rate log2 e) sp}
      }
    }
  }
  if (tg < TGN) {
#pragma unroll
    for (int j = 0; j < 8; ++j) s_tot[tg * K + i0 + j] = acc[j];
  }
  __syncthreads();
  group_prefix_excl(s_tot, K, TGN, tid);
  float off[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (tg < TGN) load8<float>(s_tot + tg * K + i0, off);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int t = tg * TPG + u;
    if (u < TPG && t < L) {
      float y[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = (off[j] + pre[u][j]) * KDN_LOG2E;
      store8<float>(g_cumsum + (((int64_t)b * T + t0 + t) * H + h) * K + i0, y);
    }
    // a = mean over channels of e^{2g}: reduce over the CG consecutive lanes of this token group
    float s = e2[u];
    if (CG == 16) {
      s = row16_sum(s);  // the same butterfly on DPP
    } else {
      for (int o = 1; o < CG; o <<= 1) s += __shfl_xor(s, o, 64);
    }
    if (cg == 0 && u < TPG && t < L) {
      const float at = s * (1.f / (float)K);  // K is a power of two: exact
      a_out[((int64_t)b * T + t0 + t) * H + h] = at;
      if (MAPS) s_ga[t] = at;
    }
  }
  if (blockIdx.x < H && tid == 0) mu_out[h] = 0.1f + fsoftplus(mu_param[h]);
  if (MAPS) {
    __syncthreads();
    if (tid < kIsoChunk) {  // wave 0, lane = token
      const Map2 M = wave_chunk_map(tid < L ? token_map(s_ga[tid], om_t, r_t, gain_s) : map_identity());
      if (tid == 0) gain_maps[((int64_t)b * H + h) * NT + nt] = float4{M.m0, M.m1, M.m2, M.m3};
    }
  }
}

// grid (H * B * NT) with the head fastest, block 256.  Per-block partials as in iso_gate_bwd_kernel.
// With GAIN (chunk = 64, the fused front) the cotangents of a, omega, r are not inputs: wave 0 runs the
// gain's backward over this chunk of (b, h) from G (reverse chunk maps, the gain's saved state) and
// hands each token's to the gate's math below.
template <typename TG, typename TO, bool GAIN>
__global__ __launch_bounds__(256) void iso_gate_bwd_vec_kernel(
    const TG* __restrict__ g_raw, const TO* __restrict__ orr, int64_t orr_sb, int64_t orr_st,
    const float* __restrict__ omega_bias, const float* __restrict__ r_bias, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, const float* __restrict__ dg_pre, const float* __restrict__ da,
    const float* __restrict__ domega, const float* __restrict__ dr, int T, int H, int K, int chunk, int NT,
    TG* __restrict__ dg_raw, TO* __restrict__ dorr, float* __restrict__ part_A, float* __restrict__ part_dt,
    float* __restrict__ part_bias, IsoGainBwdArgs G) {
  __shared__ __attribute__((aligned(16))) float s_tot[256 * 8];
  __shared__ float s_da[256];
  __shared__ float red[16];
  const int CG = K / 8, TGN = 256 / CG, TPG = (chunk + TGN - 1) / TGN;
  const int h = blockIdx.x % H, b = blockIdx.x / H / NT, nt = blockIdx.x / H % NT, tid = threadIdx.x;
  const int cg = tid % CG, tg = tid / CG, i0 = 8 * cg;
  const int t0 = nt * chunk, L = min(chunk, T - t0);
  const int p = blockIdx.x / H;
  const float rate = __expf(A_log[h]);  // once per thread
  float bias[8];
  load8<float>(dt_bias + h * K + i0, bias);
  // per-token scalars: thread tid owns token tid (chunk <= 256; loads clamped to the chunk, only
  // tid < L is used), so each is loaded once rather than by every channel group
  const int64_t srow = ((int64_t)b * T + t0 + min(tid, L - 1)) * H + h;
  float da_t = 0.f, do_t = 0.f, dr_t = 0.f;
  if (!GAIN) {
    da_t = da ? da[srow] : 0.f;
    do_t = domega ? domega[srow] : 0.f;
    dr_t = dr ? dr[srow] : 0.f;
  }
  const bool has_da = GAIN || da, has_do = GAIN || domega, has_dr = GAIN || dr;  // GAIN: all present
  const int64_t sro = (int64_t)b * orr_sb + (int64_t)(t0 + min(tid, L - 1)) * orr_st + h;
  const float or_t = ld(orr, sro), rr_t = ld(orr, sro + H);
  // every vector load of this thread's tokens goes out first (rows clamped to the chunk; the
  // clamped duplicates are never used), so the thread waits for memory once
  float dgr_in[4][8], xr[4][8];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int t = min(tg * TPG + u, L - 1);
    const int64_t row = ((int64_t)b * T + t0 + t) * H + h;
    if (dg_pre) load8<float>(dg_pre + row * K + i0, dgr_in[u]);
    load8<TG>(g_raw + row * K + i0, xr[u]);
  }
  if (GAIN && tid < kIsoChunk) iso_gain_bwd_chunk(G, b, nt, h, T, H, L, da_t, do_t, dr_t);
  s_da[tid] = da_t * (2.f / (float)K);
  // local suffix sums of dg_pre over this thread's tokens (last token first)
  float dgp[4][8], acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 3; u >= 0; --u) {
    const int t = tg * TPG + u;
#pragma unroll
    for (int j = 0; j < 8; ++j) dgp[u][j] = 0.f;
    if (dg_pre && u < TPG && t < L) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        acc[j] += dgr_in[u][j];
        dgp[u][j] = acc[j];
      }
    }
  }
  if (tg < TGN) {
#pragma unroll
    for (int j = 0; j < 8; ++j) s_tot[tg * K + i0 + j] = acc[j];
  }
  __syncthreads();
  group_suffix_excl(s_tot, K, TGN, tid);
  float off[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (tg < TGN) load8<float>(s_tot + tg * K + i0, off);
  __syncthreads();  // s_tot is reused for the per-channel ddt partials below
  float ddt[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, dA_term = 0.f, dob = 0.f, drb = 0.f;
  const float c2g = -2.f * rate * KDN_LOG2E;  // e^{2 g} for g = -rate sp is 2^{c2g sp}
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int t = tg * TPG + u;
    if (u < TPG && t < L) {
      const int64_t row = ((int64_t)b * T + t0 + t) * H + h;
      float dgr[8];
      const float dau = s_da[t];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float xb = xr[u][j] + bias[j];
        float sp, sg;
        fsoftplus_sigmoid(xb, sp, sg);
        const float g = -rate * sp;
        float dgl = dg_pre ? off[j] + dgp[u][j] : 0.f;
        if (has_da) dgl += dau * fexp2(sp * c2g);  // e^{2 g}
        dgr[j] = dgl * (-rate) * sg;
        dA_term += dgl * g;
        ddt[j] += dgr[j];
      }
      if (dg_raw) store8<TG>(dg_raw + row * K + i0, dgr);
    }
  }
  if (tid < L) {  // the per-token omega / r terms of token tid
    const float ob = has_do ? do_t * fsigmoid(or_t + omega_bias[h]) : 0.f;
    const float rb = has_dr ? dr_t * fsigmoid(rr_t + r_bias[h]) : 0.f;
    dob = ob;
    drb = rb;
    if (dorr) {
      const int64_t wo = ((int64_t)b * T + t0 + tid) * (2 * H) + h;
      st(dorr, wo, ob);
      st(dorr, wo + H, rb);
    }
  }
  // per-channel ddt partial: sum over token groups
  if (tg < TGN) {
#pragma unroll
    for (int j = 0; j < 8; ++j) s_tot[tg * K + i0 + j] = ddt[j];
  }
  __syncthreads();
  if (part_dt && tid < K) {
    float sdt = 0.f;
    for (int q = 0; q < TGN; ++q) sdt += s_tot[q * K + tid];
    part_dt[((int64_t)p * H + h) * K + tid] = sdt;
  }
  // the three block sums share one exchange: each wave's sums (xor butterflies), then the waves' in
  // order, as block_sum forms each
  const float wA = wave_sum(dA_term), wO = wave_sum(dob), wR = wave_sum(drb);
  if ((tid & 63) == 0) {
    red[3 * (tid >> 6)] = wA;
    red[3 * (tid >> 6) + 1] = wO;
    red[3 * (tid >> 6) + 2] = wR;
  }
  __syncthreads();
  if (tid == 0) {
    float sA = 0.f, sO = 0.f, sR = 0.f;
    for (int i = 0; i < 4; ++i) {
      sA += red[3 * i];
      sO += red[3 * i + 1];
      sR += red[3 * i + 2];
    }
    if (part_A) part_A[(int64_t)p * H + h] = sA;
    if (part_bias) {
      part_bias[(int64_t)p * 2 * H + h] = sO;
      part_bias[(int64_t)p * 2 * H + H + h] = sR;
    }
  }
}

__global__ void mu_fwd_kernel(const float* __restrict__ mu_param, int H, float* __restrict__ mu) {
  const int h = blockIdx.x * blockDim.x + threadIdx.x;
  if (h < H) mu[h] = 0.1f + softplusf(mu_param[h]);
}

template <typename T>
__global__ void fill_zero_kernel(T* __restrict__ p, int64_t n) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j < n) p[j] = (T)0;
}

// dmu_param = dmu * sigmoid(mu_param)
__global__ void mu_vjp_kernel(const float* __restrict__ mu_param, const float* __restrict__ dmu, int H,
                              float* __restrict__ dmu_param) {
  const int h = blockIdx.x * blockDim.x + threadIdx.x;
  if (h < H) dmu_param[h] = dmu ? dmu[h] * sigmoidf(mu_param[h]) : 0.f;
}

// ---------------------------------------------------------------------------
// Row normalisations.  One wave per row, K <= 256 (4 elements per lane).
// ---------------------------------------------------------------------------
template <typename TX, typename TY>
__global__ __launch_bounds__(256) void l2norm_fwd_kernel(const TX* __restrict__ x, int64_t rows, int K, float eps,
                                                         TY* __restrict__ y, float* __restrict__ rstd) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  float v[4];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = lane + 64 * j;
    v[j] = c < K ? ld(x, row * K + c) : 0.f;
    ss += v[j] * v[j];
  }
  ss = wave_sum(ss);
  const float rs = 1.f / sqrtf(ss + eps);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = lane + 64 * j;
    if (c < K) st(y, row * K + c, v[j] * rs);
  }
  if (lane == 0) rstd[row] = rs;
}

template <typename TX, typename TD>
__global__ __launch_bounds__(256) void l2norm_bwd_kernel(const TX* __restrict__ x, const float* __restrict__ rstd,
                                                         const TD* __restrict__ dy, int64_t rows, int K,
                                                         TX* __restrict__ dx) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float rs = rstd[row];
  float yv[4], gv[4];
  float dot = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = lane + 64 * j;
    yv[j] = c < K ? ld(x, row * K + c) * rs : 0.f;
    gv[j] = c < K ? ld(dy, row * K + c) : 0.f;
    dot += yv[j] * gv[j];
  }
  dot = wave_sum(dot);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = lane + 64 * j;
    if (c < K) st(dx, row * K + c, rs * (gv[j] - yv[j] * dot));
  }
}

// Vectorised row kernels: LPR = K/8 lanes per row, each lane 8 consecutive elements.
template <typename TX, typename TY>
__global__ __launch_bounds__(256) void l2norm_fwd_vec_kernel(const TX* __restrict__ x, int64_t rows, int K, float eps,
                                                             TY* __restrict__ y, float* __restrict__ rstd) {
  const int LPR = K / 8, RPB = 256 / LPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR;
  const int sub = threadIdx.x % LPR;
  float v[8];
  float ss = 0.f;
  if (row < rows) {
    load8<TX>(x + row * K + 8 * sub, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += v[j] * v[j];
  }
  for (int o = 1; o < LPR; o <<= 1) ss += __shfl_xor(ss, o, 64);
  if (row >= rows) return;
  const float rs = 1.f / sqrtf(ss + eps);
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] *= rs;
  store8<TY>(y + row * K + 8 * sub, v);
  if (sub == 0) rstd[row] = rs;
}

template <typename TX, typename TD>
__global__ __launch_bounds__(256) void l2norm_bwd_vec_kernel(const TX* __restrict__ x, const float* __restrict__ rstd,
                                                             const TD* __restrict__ dy, int64_t rows, int K,
                                                             TX* __restrict__ dx) {
  const int LPR = K / 8, RPB = 256 / LPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR;
  const int sub = threadIdx.x % LPR;
  float yv[8], gv[8];
  float dot = 0.f, rs = 0.f;
  if (row < rows) {
    rs = rstd[row];
    load8<TX>(x + row * K + 8 * sub, yv);
    load8<TD>(dy + row * K + 8 * sub, gv);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      yv[j] *= rs;
      dot += yv[j] * gv[j];
    }
  }
  for (int o = 1; o < LPR; o <<= 1) dot += __shfl_xor(dot, o, 64);
  if (row >= rows) return;
  float d[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) d[j] = rs * (gv[j] - yv[j] * dot);
  store8<TX>(dx + row * K + 8 * sub, d);
}

// diag normalisation: y = x / max(||x||, 1e-12).  Emits q bf16, k fp32 (gain), k bf16 (memory).
template <typename TX>
__global__ __launch_bounds__(256) void diag_norm_fwd_kernel(const TX* __restrict__ q, const TX* __restrict__ k,
                                                            int64_t rows, int K, bf16_t* __restrict__ q_mem,
                                                            float* __restrict__ k_gain, bf16_t* __restrict__ k_mem,
                                                            float* __restrict__ q_norm, float* __restrict__ k_norm) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  float qv[4], kv[4], sq = 0.f, sk = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = lane + 64 * j;
    qv[j] = c < K ? ld(q, row * K + c) : 0.f;
    kv[j] = c < K ? ld(k, row * K + c) : 0.f;
    sq += qv[j] * qv[j];
    sk += kv[j] * kv[j];
  }
  const float nq = sqrtf(wave_sum(sq)), nk = sqrtf(wave_sum(sk));
  const float dq = fmaxf(nq, 1e-12f), dk = fmaxf(nk, 1e-12f);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = lane + 64 * j;
    if (c < K) {
      q_mem[row * K + c] = f2bf(qv[j] / dq);
      const float kn = kv[j] / dk;
      if (k_gain) k_gain[row * K + c] = kn;
      k_mem[row * K + c] = f2bf(kn);
    }
  }
  if (lane == 0) {
    q_norm[row] = nq;
    k_norm[row] = nk;
  }
}

// Row VJP of y = x / max(||x||, eps): n > eps: (dy - y (y.dy)) / n; else dy / eps.
template <typename TX>
__device__ __forceinline__ void norm_row_vjp(const TX* x, float n, const float* g, int64_t row, int K, int lane,
                                             TX* dx) {
  const float d = fmaxf(n, 1e-12f);
  float yv[4], dot = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = lane + 64 * j;
    yv[j] = c < K ? ld(x, row * K + c) / d : 0.f;
    dot += yv[j] * g[j];
  }
  dot = wave_sum(dot);
  const bool clamped = !(n > 1e-12f);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = lane + 64 * j;
    if (c < K) st(dx, row * K + c, clamped ? g[j] / d : (g[j] - yv[j] * dot) / d);
  }
}

template <typename TX>
__global__ __launch_bounds__(256) void diag_norm_bwd_kernel(
    const TX* __restrict__ q, const TX* __restrict__ k, const float* __restrict__ q_norm,
    const float* __restrict__ k_norm, const bf16_t* __restrict__ dq_mem, const float* __restrict__ dk_gain,
    const bf16_t* __restrict__ dk_mem, int64_t rows, int K, TX* __restrict__ dq, TX* __restrict__ dk) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  float g[4];
  if (dq) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = lane + 64 * j;
      g[j] = (c < K && dq_mem) ? bf2f(dq_mem[row * K + c]) : 0.f;
    }
    norm_row_vjp(q, q_norm[row], g, row, K, lane, dq);
  }
  if (dk) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = lane + 64 * j;
      float s = 0.f;
      if (c < K) {
        if (dk_gain) s += dk_gain[row * K + c];
        if (dk_mem) s += bf2f(dk_mem[row * K + c]);
      }
      g[j] = s;
    }
    norm_row_vjp(k, k_norm[row], g, row, K, lane, dk);
  }
}

// ---------------------------------------------------------------------------
// diag frontend.  grid (H * B * NT) with the head fastest, block 256 (thread = key channel).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void diag_frontend_fwd_kernel(
    const bf16_t* __restrict__ f_raw, const bf16_t* __restrict__ z_raw, const bf16_t* __restrict__ y_raw,
    const float* __restrict__ A_log, const float* __restrict__ dt_bias, const float* __restrict__ mu_param, int T,
    int H, int K, int chunk, int NT, float* __restrict__ g_cumsum, float* __restrict__ alpha,
    float* __restrict__ omega, float* __restrict__ r, float* __restrict__ mu) {
  const int h = blockIdx.x % H, b = blockIdx.x / H / NT, nt = blockIdx.x / H % NT, i = threadIdx.x;
  const int t0 = nt * chunk, L = min(chunk, T - t0);
  const float rate = __expf(A_log[h]);
  const float floor_log = logf(1e-6f);
  if (i < K) {
    const float bias = dt_bias[h * K + i];
    float acc = 0.f;
    for (int t = 0; t < L; ++t) {
      const int64_t off = (((int64_t)b * T + t0 + t) * H + h) * K + i;
      const float ell = -rate * softplusf(bf2f(f_raw[off]) + bias);
      const float al = expf(ell);
      // memory path clamps alpha at 1e-6 (NaN propagates)
      const float ell_mem = (al >= 1e-6f || al != al) ? ell : floor_log;
      acc += ell_mem;
      g_cumsum[off] = acc * KDN_LOG2E;
      alpha[off] = al;
      omega[off] = softplusf(bf2f(z_raw[off]));
    }
  }
  if (i < L) {
    const int64_t o = ((int64_t)b * T + t0 + i) * H + h;
    r[o] = 0.01f + softplusf(bf2f(y_raw[o]));
  }
  if (blockIdx.x < H && i == 0) mu[h] = 0.1f + softplusf(mu_param[h]);
}

__global__ __launch_bounds__(256) void diag_frontend_bwd_kernel(
    const bf16_t* __restrict__ f_raw, const float* __restrict__ A_log, const float* __restrict__ dt_bias,
    const float* __restrict__ alpha, const float* __restrict__ dG, const float* __restrict__ dalpha, int T, int H,
    int K, int chunk, int NT, bf16_t* __restrict__ df_raw, float* __restrict__ part_A,
    float* __restrict__ part_dt) {
  __shared__ float red[16];
  const int h = blockIdx.x % H, b = blockIdx.x / H / NT, nt = blockIdx.x / H % NT, i = threadIdx.x;
  const int t0 = nt * chunk, L = min(chunk, T - t0);
  const int p = blockIdx.x / H;
  const float rate = __expf(A_log[h]);
  float dA_term = 0.f;
  if (i < K) {
    const float bias = dt_bias[h * K + i];
    float acc = 0.f, ddt = 0.f;
    for (int t = L - 1; t >= 0; --t) {
      const int64_t off = (((int64_t)b * T + t0 + t) * H + h) * K + i;
      const float x = bf2f(f_raw[off]) + bias;
      const float ell = -rate * softplusf(x);
      const float al = alpha[off];
      float dell = 0.f;
      if (dG) {
        acc += dG[off];
        if (al >= 1e-6f) dell = acc;
      }
      if (dalpha) dell += dalpha[off] * al;
      const float df = dell * (-rate) * sigmoidf(x);
      if (df_raw) df_raw[off] = f2bf(df);
      dA_term += dell * ell;
      ddt += df;
    }
    if (part_dt) part_dt[((int64_t)p * H + h) * K + i] = ddt;
  }
  const float sA = block_sum(dA_term, red);
  if (part_A && i == 0) part_A[(int64_t)p * H + h] = sA;
}

// ---------------------------------------------------------------------------
// Vectorised diag frontend (same thread layout as the vectorised iso gate).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void diag_frontend_fwd_vec_kernel(
    const bf16_t* __restrict__ f_raw, const bf16_t* __restrict__ z_raw, const bf16_t* __restrict__ y_raw,
    const float* __restrict__ A_log, const float* __restrict__ dt_bias, const float* __restrict__ mu_param, int T,
    int H, int K, int chunk, int NT, float* __restrict__ g_cumsum, float* __restrict__ alpha,
    float* __restrict__ omega, float* __restrict__ r, float* __restrict__ mu) {
  __shared__ float s_tot[256 * 8];
  const int CG = K / 8, TGN = 256 / CG, TPG = (chunk + TGN - 1) / TGN;
  const int h = blockIdx.x % H, b = blockIdx.x / H / NT, nt = blockIdx.x / H % NT, tid = threadIdx.x;
  const int cg = tid % CG, tg = tid / CG, i0 = 8 * cg;
  const int t0 = nt * chunk, L = min(chunk, T - t0);
  const float rate = __expf(A_log[h]);
  const float floor_log = -13.815510557964274f;  // log(1e-6)
  float bias[8];
  load8<float>(dt_bias + h * K + i0, bias);
  // the loads of all this thread's tokens go out first (rows clamped to the chunk)
  float xr[4][8], zrr[4][8];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t off = (((int64_t)b * T + t0 + min(tg * TPG + u, L - 1)) * H + h) * K + i0;
    load8<bf16_t>(f_raw + off, xr[u]);
    load8<bf16_t>(z_raw + off, zrr[u]);
  }
  const float yv = tid < L ? bf2f(y_raw[((int64_t)b * T + t0 + tid) * H + h]) : 0.f;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float pre[4][8];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int t = tg * TPG + u;
    if (u < TPG && t < L) {
      const int64_t off = (((int64_t)b * T + t0 + t) * H + h) * K + i0;
      float al[8], om[8];
      const float* x = xr[u];
      const float* zr = zrr[u];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float ell = -rate * softplusf(x[j] + bias[j]);
        al[j] = __expf(ell);
        // memory path clamps alpha at 1e-6 (NaN propagates)
        acc[j] += (al[j] >= 1e-6f || al[j] != al[j]) ? ell : floor_log;
        pre[u][j] = acc[j];
        om[j] = softplusf(zr[j]);
      }
      store8<float>(alpha + off, al);
      store8<float>(omega + off, om);
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) s_tot[tg * K + i0 + j] = acc[j];
  __syncthreads();
  float offs[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int q = 0; q < tg; ++q)
#pragma unroll
    for (int j = 0; j < 8; ++j) offs[j] += s_tot[q * K + i0 + j];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int t = tg * TPG + u;
    if (u < TPG && t < L) {
      float y[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = (offs[j] + pre[u][j]) * KDN_LOG2E;
      store8<float>(g_cumsum + (((int64_t)b * T + t0 + t) * H + h) * K + i0, y);
    }
  }
  if (tid < L) r[((int64_t)b * T + t0 + tid) * H + h] = 0.01f + softplusf(yv);
  if (blockIdx.x < H && tid == 0) mu[h] = 0.1f + softplusf(mu_param[h]);
}

__global__ __launch_bounds__(256) void diag_frontend_bwd_vec_kernel(
    const bf16_t* __restrict__ f_raw, const float* __restrict__ A_log, const float* __restrict__ dt_bias,
    const float* __restrict__ alpha, const float* __restrict__ dG, const float* __restrict__ dalpha, int T, int H,
    int K, int chunk, int NT, bf16_t* __restrict__ df_raw, float* __restrict__ part_A,
    float* __restrict__ part_dt) {
  __shared__ float s_tot[256 * 8];
  __shared__ float red[16];
  const int CG = K / 8, TGN = 256 / CG, TPG = (chunk + TGN - 1) / TGN;
  const int h = blockIdx.x % H, b = blockIdx.x / H / NT, nt = blockIdx.x / H % NT, tid = threadIdx.x;
  const int cg = tid % CG, tg = tid / CG, i0 = 8 * cg;
  const int t0 = nt * chunk, L = min(chunk, T - t0);
  const int p = blockIdx.x / H;
  const float rate = __expf(A_log[h]);
  float bias[8];
  load8<float>(dt_bias + h * K + i0, bias);
  // the loads of all this thread's tokens go out first (rows clamped to the chunk); alpha is
  // recomputed from f_raw with the forward's own operations (bit-identical), not read back
  float dGr[4][8], xr[4][8], dar[4][8];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t off = (((int64_t)b * T + t0 + min(tg * TPG + u, L - 1)) * H + h) * K + i0;
    if (dG) load8<float>(dG + off, dGr[u]);
    load8<bf16_t>(f_raw + off, xr[u]);
    if (dalpha) load8<float>(dalpha + off, dar[u]);
  }
  // local suffix sums of dG over this thread's tokens
  float dgs[4][8], acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 3; u >= 0; --u) {
    const int t = tg * TPG + u;
#pragma unroll
    for (int j = 0; j < 8; ++j) dgs[u][j] = 0.f;
    if (dG && u < TPG && t < L) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        acc[j] += dGr[u][j];
        dgs[u][j] = acc[j];
      }
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) s_tot[tg * K + i0 + j] = acc[j];
  __syncthreads();
  float offs[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int q = tg + 1; q < TGN; ++q)
#pragma unroll
    for (int j = 0; j < 8; ++j) offs[j] += s_tot[q * K + i0 + j];
  __syncthreads();
  float ddt[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, dA_term = 0.f;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int t = tg * TPG + u;
    if (u < TPG && t < L) {
      const int64_t off = (((int64_t)b * T + t0 + t) * H + h) * K + i0;
      float df[8];
      const float* x = xr[u];
      const float* da = dar[u];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float xb = x[j] + bias[j];
        float sp, sg;
        softplus_sigmoid(xb, sp, sg);
        const float ell = -rate * sp;
        const float al = __expf(ell);
        float dell = (dG && al >= 1e-6f) ? offs[j] + dgs[u][j] : 0.f;
        if (dalpha) dell += da[j] * al;
        df[j] = dell * (-rate) * sg;
        dA_term += dell * ell;
        ddt[j] += df[j];
      }
      if (df_raw) store8<bf16_t>(df_raw + off, df);
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) s_tot[tg * K + i0 + j] = ddt[j];
  __syncthreads();
  if (part_dt && tid < K) {
    float sdt = 0.f;
    for (int q = 0; q < TGN; ++q) sdt += s_tot[q * K + tid];
    part_dt[((int64_t)p * H + h) * K + tid] = sdt;
  }
  const float sA = block_sum(dA_term, red);
  if (part_A && tid == 0) part_A[(int64_t)p * H + h] = sA;
}

// Vectorised diag normalisation rows (K/8 lanes per row, 8 elements per lane).
template <typename TX>
__global__ __launch_bounds__(256) void diag_norm_fwd_vec_kernel(const TX* __restrict__ q, const TX* __restrict__ k,
                                                                int64_t rows, int K, bf16_t* __restrict__ q_mem,
                                                                float* __restrict__ k_gain, bf16_t* __restrict__ k_mem,
                                                                float* __restrict__ q_norm,
                                                                float* __restrict__ k_norm) {
  const int LPR = K / 8, RPB = 256 / LPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR;
  const int sub = threadIdx.x % LPR;
  float qv[8], kv[8], sq = 0.f, sk = 0.f;
  if (row < rows) {
    load8<TX>(q + row * K + 8 * sub, qv);
    load8<TX>(k + row * K + 8 * sub, kv);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      sq += qv[j] * qv[j];
      sk += kv[j] * kv[j];
    }
  }
  for (int o = 1; o < LPR; o <<= 1) {
    sq += __shfl_xor(sq, o, 64);
    sk += __shfl_xor(sk, o, 64);
  }
  if (row >= rows) return;
  const float nq = sqrtf(sq), nk = sqrtf(sk);
  const float iq = 1.f / fmaxf(nq, 1e-12f), ik = 1.f / fmaxf(nk, 1e-12f);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    qv[j] *= iq;
    kv[j] *= ik;
  }
  store8<bf16_t>(q_mem + row * K + 8 * sub, qv);
  if (k_gain) store8<float>(k_gain + row * K + 8 * sub, kv);  // null: the fused gain recomputes it
  store8<bf16_t>(k_mem + row * K + 8 * sub, kv);
  if (sub == 0) {
    q_norm[row] = nq;
    k_norm[row] = nk;
  }
}

// Row VJP of y = x / max(||x||, eps) on 8 elements per lane, LPR lanes per row.
template <typename TX>
__device__ __forceinline__ void norm_row_vjp8(const TX* x, float n, const float* g, int LPR, bool valid, float* dx) {
  const float d = fmaxf(n, 1e-12f), id = 1.f / d;
  float yv[8], dot = 0.f;
  if (valid) {
    load8<TX>(x, yv);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      yv[j] *= id;
      dot += yv[j] * g[j];
    }
  }
  for (int o = 1; o < LPR; o <<= 1) dot += __shfl_xor(dot, o, 64);
  const bool clamped = !(n > 1e-12f);
#pragma unroll
  for (int j = 0; j < 8; ++j) dx[j] = clamped ? g[j] * id : (g[j] - yv[j] * dot) * id;
}

template <typename TX>
__global__ __launch_bounds__(256) void diag_norm_bwd_vec_kernel(
    const TX* __restrict__ q, const TX* __restrict__ k, const float* __restrict__ q_norm,
    const float* __restrict__ k_norm, const bf16_t* __restrict__ dq_mem, const float* __restrict__ dk_gain,
    const bf16_t* __restrict__ dk_mem, int64_t rows, int K, TX* __restrict__ dq, TX* __restrict__ dk) {
  const int LPR = K / 8, RPB = 256 / LPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR;
  const int sub = threadIdx.x % LPR;
  const bool valid = row < rows;
  const int64_t e = (valid ? row : 0) * K + 8 * sub;
  float g[8], out[8];
  if (dq) {
#pragma unroll
    for (int j = 0; j < 8; ++j) g[j] = 0.f;
    if (valid && dq_mem) load8<bf16_t>(dq_mem + e, g);
    norm_row_vjp8<TX>(q + e, valid ? q_norm[row] : 1.f, g, LPR, valid, out);
    if (valid) store8<TX>(dq + e, out);
  }
  if (dk) {
    float g2[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) g[j] = 0.f;
    if (valid && dk_gain) load8<float>(dk_gain + e, g);
    if (valid && dk_mem) {
      load8<bf16_t>(dk_mem + e, g2);
#pragma unroll
      for (int j = 0; j < 8; ++j) g[j] += g2[j];
    }
    norm_row_vjp8<TX>(k + e, valid ? k_norm[row] : 1.f, g, LPR, valid, out);
    if (valid) store8<TX>(dk + e, out);
  }
}

// d raw = d * sigmoid(raw) for the (optional) omega / r cotangents reaching the frontend.
__global__ void sigmoid_vjp_kernel(const bf16_t* __restrict__ raw, const float* __restrict__ d, int64_t n,
                                   bf16_t* __restrict__ out) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j < n) out[j] = f2bf(d[j] * sigmoidf(bf2f(raw[j])));
}

inline int cdiv(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

}  // namespace

// The vectorised gate kernels need 8-channel groups that tile 256 threads, at most 4 tokens per
// thread, and 16-byte aligned rows.
inline bool aligned16(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool gate_vec_ok(int K, int chunk) {  // the vector kernels also give each of the chunk's
  if (K % 8 != 0 || 256 % (K / 8) != 0) return false;  // tokens one thread: chunk <= 256
  return chunk <= 4 * (256 / (K / 8)) && chunk <= 256;
}
// Row kernels: K/8 lanes per row, 8 elements per lane (K/8 a power of two dividing 64).
inline bool row_vec_ok(int K) { return K % 8 == 0 && K <= 512 && 64 % (K / 8) == 0; }

// The fused iso front's workspace parts (see kdn_iso_front_workspace_size).
struct IsoFrontWs {
  float* gate;
  size_t gate_bytes;
  void* gain;
  size_t gain_bytes;
  float* rows;
  float* grads;
};
inline size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }
inline IsoFrontWs iso_front_ws(void* ws, int B, int T, int H, int K) {
  IsoFrontWs w;
  char* p = (char*)ws;
  w.gate = (float*)p;
  w.gate_bytes = kdn_iso_gate_bwd_workspace_size(B, T, H, K, kIsoChunk);
  p += al256(w.gate_bytes);
  w.gain = p;
  w.gain_bytes = kdn_iso_gain_workspace_size(B, T, H);
  p += al256(w.gain_bytes);
  w.rows = (float*)p;
  p += al256((size_t)B * H * sizeof(float));
  w.grads = (float*)p;
  return w;
}

// ============================================================================
// C ABI
// ============================================================================
extern "C" {

size_t kdn_iso_gate_bwd_workspace_size(int B, int T, int H, int K, int chunk) {
  const int64_t NP = (int64_t)B * cdiv(T, chunk);
  return (size_t)(NP * H + NP * H * K + NP * 2 * H) * sizeof(float);
}

int kdn_iso_gate_fwd(const void* g_raw, int g_raw_bf16, const void* omega_r_raw, int orr_bf16, int64_t orr_stride_b,
                     int64_t orr_stride_t, const float* omega_bias, const float* r_bias, const float* A_log,
                     const float* dt_bias, const float* mu_param, float omega_min, float r_min, int B, int T, int H,
                     int K, int chunk, float* g_cumsum, float* a, float* omega, float* r, float* mu,
                     hipStream_t stream) {
  if (K <= 0 || K > 256 || chunk <= 0 || chunk > kMaxChunk || B < 0 || T < 0 || H <= 0) return KDN_ERR_ARG;
  if (B == 0 || T == 0) {
    hipLaunchKernelGGL(mu_fwd_kernel, dim3(cdiv(H, 256)), dim3(256), 0, stream, mu_param, H, mu);
    KDN_CHECK_LAUNCH();
    return 0;
  }
  const int NT = cdiv(T, chunk);
  // head fastest: the workgroups in flight read neighbouring heads' rows of the same tokens
  dim3 grid(H * B * NT);
  const bool vec = gate_vec_ok(K, chunk) && aligned16(g_raw) && aligned16(g_cumsum) && aligned16(dt_bias);
#define KDN_GATE_FWD(TG, TO)                                                                                     \
  if (vec)                                                                                                       \
    hipLaunchKernelGGL((iso_gate_fwd_vec_kernel<TG, TO, false>), grid, dim3(256), 0, stream, (const TG*)g_raw,    \
                       (const TO*)omega_r_raw, orr_stride_b, orr_stride_t, omega_bias, r_bias, A_log, dt_bias,   \
                       mu_param, omega_min, r_min, T, H, K, chunk, NT, g_cumsum, a, omega, r, mu, nullptr, 0.f); \
  else                                                                                                           \
    hipLaunchKernelGGL((iso_gate_fwd_kernel<TG, TO>), grid, dim3(256), 0, stream, (const TG*)g_raw,              \
                       (const TO*)omega_r_raw, orr_stride_b, orr_stride_t, omega_bias, r_bias, A_log, dt_bias,   \
                       mu_param, omega_min, r_min, T, H, K, chunk, NT, g_cumsum, a, omega, r, mu)
  if (g_raw_bf16 && orr_bf16) KDN_GATE_FWD(bf16_t, bf16_t);
  else if (g_raw_bf16) KDN_GATE_FWD(bf16_t, float);
  else if (orr_bf16) KDN_GATE_FWD(float, bf16_t);
  else KDN_GATE_FWD(float, float);
#undef KDN_GATE_FWD
  KDN_CHECK_LAUNCH();
  return 0;
}

int kdn_iso_gate_bwd(const void* g_raw, int g_raw_bf16, const void* omega_r_raw, int orr_bf16, int64_t orr_stride_b,
                     int64_t orr_stride_t, const float* omega_bias, const float* r_bias, const float* A_log,
                     const float* dt_bias, const float* mu_param, const float* dg_pre, const float* da,
                     const float* domega, const float* dr, const float* dmu, int B, int T, int H, int K, int chunk,
                     void* dg_raw, void* domega_r_raw, float* dA_log, float* ddt_bias, float* domega_bias,
                     float* dr_bias, float* dmu_param, void* workspace, size_t workspace_bytes,
                     hipStream_t stream) {
  if (K <= 0 || K > 256 || chunk <= 0 || chunk > kMaxChunk || B <= 0 || T <= 0 || H <= 0) return KDN_ERR_ARG;
  if (workspace_bytes < kdn_iso_gate_bwd_workspace_size(B, T, H, K, chunk)) return KDN_ERR_ARG;
  const int NT = cdiv(T, chunk);
  const int NP = B * NT;
  float* part_A = (float*)workspace;
  float* part_dt = part_A + (int64_t)NP * H;
  float* part_bias = part_dt + (int64_t)NP * H * K;
  dim3 grid(H * NP);  // head fastest
  const bool vec = gate_vec_ok(K, chunk) && aligned16(g_raw) && aligned16(dg_pre) && aligned16(dg_raw) &&
                   aligned16(dt_bias);
#define KDN_GATE_BWD(TG, TO)                                                                                     \
  if (vec)                                                                                                       \
    hipLaunchKernelGGL((iso_gate_bwd_vec_kernel<TG, TO, false>), grid, dim3(256), 0, stream, (const TG*)g_raw,    \
                       (const TO*)omega_r_raw, orr_stride_b, orr_stride_t, omega_bias, r_bias, A_log, dt_bias,   \
                       dg_pre, da, domega, dr, T, H, K, chunk, NT, (TG*)dg_raw, (TO*)domega_r_raw,               \
                       dA_log ? part_A : nullptr, ddt_bias ? part_dt : nullptr,                                  \
                       (domega_bias || dr_bias) ? part_bias : nullptr, IsoGainBwdArgs{});                        \
  else                                                                                                           \
    hipLaunchKernelGGL((iso_gate_bwd_kernel<TG, TO>), grid, dim3(256), 0, stream, (const TG*)g_raw,              \
                       (const TO*)omega_r_raw, orr_stride_b, orr_stride_t, omega_bias, r_bias, A_log, dt_bias,   \
                       dg_pre, da, domega, dr, T, H, K, chunk, NT, (TG*)dg_raw, (TO*)domega_r_raw,               \
                       dA_log ? part_A : nullptr, ddt_bias ? part_dt : nullptr,                                  \
                       (domega_bias || dr_bias) ? part_bias : nullptr)
  if (g_raw_bf16 && orr_bf16) KDN_GATE_BWD(bf16_t, bf16_t);
  else if (g_raw_bf16) KDN_GATE_BWD(bf16_t, float);
  else if (orr_bf16) KDN_GATE_BWD(float, bf16_t);
  else KDN_GATE_BWD(float, float);
#undef KDN_GATE_BWD
  KDN_CHECK_LAUNCH();
  // the parameter gradients' partial sums and the prior-precision VJP, one launch
  PartSegs P{};
  if (dA_log) P.seg[P.nseg++] = PartSeg{part_A, (int64_t)H, H, dA_log};
  if (ddt_bias) P.seg[P.nseg++] = PartSeg{part_dt, (int64_t)H * K, H * K, ddt_bias};
  // part_bias rows are [omega(H) | r(H)]
  if (domega_bias) P.seg[P.nseg++] = PartSeg{part_bias, (int64_t)2 * H, H, domega_bias};
  if (dr_bias) P.seg[P.nseg++] = PartSeg{part_bias + H, (int64_t)2 * H, H, dr_bias};
  P.mu_param = mu_param;
  P.dmu = dmu;
  P.H = H;
  P.dmu_param = dmu_param;
  const int nblk = part_segs_blocks(P);
  if (nblk > 0) hipLaunchKernelGGL(reduce_partials_multi_kernel, dim3(nblk), dim3(256), 0, stream, P, NP);
  KDN_CHECK_LAUNCH();
  return 0;
}

// ---------------------------------------------------------------- fused iso front
// The gate and the gain as the layer composes them.  Workspace: the gate backward's partials, the gain's
// workspace (the fused path's chunk maps), per-row prior cotangents [B*H], and the unfused path's
// a / omega / r cotangents [3][B,T,H] plus a prior cotangent [H]; each part 256-byte aligned.

size_t kdn_iso_front_workspace_size(int B, int T, int H, int K) {
  if (B <= 0 || T <= 0 || H <= 0 || K <= 0) return 0;
  return al256(kdn_iso_gate_bwd_workspace_size(B, T, H, K, kIsoChunk)) + al256(kdn_iso_gain_workspace_size(B, T, H)) +
         al256((size_t)B * H * sizeof(float)) + al256(((size_t)3 * B * T * H + H) * sizeof(float));
}

int kdn_iso_front_fwd(const void* g_raw, int g_raw_bf16, const void* omega_r_raw, int orr_bf16, int64_t orr_stride_b,
                      int64_t orr_stride_t, const float* omega_bias, const float* r_bias, const float* A_log,
                      const float* dt_bias, const float* mu_param, float omega_min, float r_min,
                      const float* initial_precision, int prec_mode, int B, int T, int H, int K, float posterior_scale,
                      float* g_cumsum, float* a, float* omega, float* r, float* mu, float* beta, float* p_prev,
                      float* final_precision, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (K <= 0 || K > 256 || B < 0 || T < 0 || H <= 0 || H > 96 || !(posterior_scale > 0.f)) return KDN_ERR_ARG;
  if ((prec_mode != 0 && prec_mode != 1) || (prec_mode == 1 && !initial_precision)) return KDN_ERR_ARG;
  if (!a || !omega || !r || !mu || !beta) return KDN_ERR_ARG;
  if (B == 0 || T == 0)  // mu only (the final precision of an empty sequence is the initial one: the caller's)
    return kdn_iso_gate_fwd(g_raw, g_raw_bf16, omega_r_raw, orr_bf16, orr_stride_b, orr_stride_t, omega_bias, r_bias,
                            A_log, dt_bias, mu_param, omega_min, r_min, B, T, H, K, kIsoChunk, g_cumsum, a, omega, r,
                            mu, stream);
  if (workspace_bytes < kdn_iso_front_workspace_size(B, T, H, K)) return KDN_ERR_ARG;
  const IsoFrontWs ws = iso_front_ws(workspace, B, T, H, K);
  const float* prior = initial_precision ? initial_precision : mu;
  const bool vec = gate_vec_ok(K, kIsoChunk) && aligned16(g_raw) && aligned16(g_cumsum) && aligned16(dt_bias);
  if (!vec) {  // the two ops one after the other
    const int rc = kdn_iso_gate_fwd(g_raw, g_raw_bf16, omega_r_raw, orr_bf16, orr_stride_b, orr_stride_t, omega_bias,
                                    r_bias, A_log, dt_bias, mu_param, omega_min, r_min, B, T, H, K, kIsoChunk,
                                    g_cumsum, a, omega, r, mu, stream);
    if (rc != 0) return rc;
    return kdn_iso_gain_fwd(a, omega, r, prior, prec_mode, B, T, H, posterior_scale, beta, p_prev, final_precision,
                            ws.gain, ws.gain_bytes, stream);
  }
  const int NC = cdiv(T, kIsoChunk);
  float4* maps = (float4*)ws.gain;
  dim3 grid(H * B * NC);
#define KDN_FRONT_FWD(TG, TO)                                                                                    \
  hipLaunchKernelGGL((iso_gate_fwd_vec_kernel<TG, TO, true>), grid, dim3(256), 0, stream, (const TG*)g_raw,      \
                     (const TO*)omega_r_raw, orr_stride_b, orr_stride_t, omega_bias, r_bias, A_log, dt_bias,     \
                     mu_param, omega_min, r_min, T, H, K, kIsoChunk, NC, g_cumsum, a, omega, r, mu, maps,       \
                     posterior_scale)
  if (g_raw_bf16 && orr_bf16) KDN_FRONT_FWD(bf16_t, bf16_t);
  else if (g_raw_bf16) KDN_FRONT_FWD(bf16_t, float);
  else if (orr_bf16) KDN_FRONT_FWD(float, bf16_t);
  else KDN_FRONT_FWD(float, float);
#undef KDN_FRONT_FWD
  launch_iso_gain_emit(a, omega, r, maps, prior, prec_mode, B, T, H, NC, posterior_scale, beta, p_prev,
                       final_precision, stream);
  KDN_CHECK_LAUNCH();
  return 0;
}

int kdn_iso_front_bwd(const void* g_raw, int g_raw_bf16, const void* omega_r_raw, int orr_bf16, int64_t orr_stride_b,
                      int64_t orr_stride_t, const float* omega_bias, const float* r_bias, const float* A_log,
                      const float* dt_bias, const float* mu_param, const float* initial_precision, int prec_mode,
                      const float* a, const float* omega, const float* r, const float* mu, const float* p_prev,
                      const float* final_precision, const float* dg_pre, const float* dbeta,
                      const float* d_final_precision, int B, int T, int H, int K, float posterior_scale, void* dg_raw,
                      void* domega_r_raw, float* dA_log, float* ddt_bias, float* domega_bias, float* dr_bias,
                      float* dmu_param, float* d_initial_precision, void* workspace, size_t workspace_bytes,
                      hipStream_t stream) {
  if (K <= 0 || K > 256 || B <= 0 || T <= 0 || H <= 0 || H > 96 || !(posterior_scale > 0.f)) return KDN_ERR_ARG;
  if ((prec_mode != 0 && prec_mode != 1) || (prec_mode == 1 && !initial_precision)) return KDN_ERR_ARG;
  if (!a || !omega || !r || !mu || !p_prev || !dbeta || (d_final_precision && !final_precision)) return KDN_ERR_ARG;
  if (workspace_bytes < kdn_iso_front_workspace_size(B, T, H, K)) return KDN_ERR_ARG;
  const IsoFrontWs ws = iso_front_ws(workspace, B, T, H, K);
  const float* prior = initial_precision ? initial_precision : mu;
  const bool vec = gate_vec_ok(K, kIsoChunk) && aligned16(g_raw) && aligned16(dg_pre) && aligned16(dg_raw) &&
                   aligned16(dt_bias);
  if (!vec) {  // the gain's backward into the workspace, then the gate's
    const int64_t n = (int64_t)B * T * H;
    float *gda = ws.grads, *gdo = gda + n, *gdr = gdo + n, *gdmu = gdr + n;
    int rc = kdn_iso_gain_bwd(a, omega, r, prior, prec_mode, dbeta, p_prev, final_precision, d_final_precision, B, T,
                              H, posterior_scale, gda, gdo, gdr, initial_precision ? d_initial_precision : gdmu,
                              ws.gain, ws.gain_bytes, stream);
    if (rc != 0) return rc;
    return kdn_iso_gate_bwd(g_raw, g_raw_bf16, omega_r_raw, orr_bf16, orr_stride_b, orr_stride_t, omega_bias, r_bias,
                            A_log, dt_bias, mu_param, dg_pre, gda, gdo, gdr, initial_precision ? nullptr : gdmu, B, T,
                            H, K, kIsoChunk, dg_raw, domega_r_raw, dA_log, ddt_bias, domega_bias, dr_bias, dmu_param,
                            ws.gate, ws.gate_bytes, stream);
  }
  const int NC = cdiv(T, kIsoChunk), NP = B * NC;
  float2* maps = (float2*)ws.gain;
  launch_iso_gain_bwd_map(a, omega, r, dbeta, p_prev, B, T, H, NC, posterior_scale, maps, stream);
  // per-row prior cotangents: the [B,H] initial precision's own (prec_mode 1), else rows summed below
  float* rows = nullptr;
  if (prec_mode == 1) rows = d_initial_precision;
  else if (initial_precision ? d_initial_precision != nullptr : dmu_param != nullptr) rows = ws.rows;
  const IsoGainBwdArgs G{maps, a, omega, r, dbeta, p_prev, final_precision, d_final_precision, prior, rows,
                         prec_mode, NC, posterior_scale == 1.f ? 1 : 0, posterior_scale};
  float* part_A = ws.gate;
  float* part_dt = part_A + (int64_t)NP * H;
  float* part_bias = part_dt + (int64_t)NP * H * K;
  dim3 grid(H * NP);  // head fastest
#define KDN_FRONT_BWD(TG, TO)                                                                                    \
  hipLaunchKernelGGL((iso_gate_bwd_vec_kernel<TG, TO, true>), grid, dim3(256), 0, stream, (const TG*)g_raw,      \
                     (const TO*)omega_r_raw, orr_stride_b, orr_stride_t, omega_bias, r_bias, A_log, dt_bias,     \
                     dg_pre, nullptr, nullptr, nullptr, T, H, K, kIsoChunk, NC, (TG*)dg_raw, (TO*)domega_r_raw,  \
                     dA_log ? part_A : nullptr, ddt_bias ? part_dt : nullptr,                                    \
                     (domega_bias || dr_bias) ? part_bias : nullptr, G)
  if (g_raw_bf16 && orr_bf16) KDN_FRONT_BWD(bf16_t, bf16_t);
  else if (g_raw_bf16) KDN_FRONT_BWD(bf16_t, float);
  else if (orr_bf16) KDN_FRONT_BWD(float, bf16_t);
  else KDN_FRONT_BWD(float, float);
#undef KDN_FRONT_BWD
  KDN_CHECK_LAUNCH();
  PartSegs P{};
  if (dA_log) P.seg[P.nseg++] = PartSeg{part_A, (int64_t)H, H, dA_log};
  if (ddt_bias) P.seg[P.nseg++] = PartSeg{part_dt, (int64_t)H * K, H * K, ddt_bias};
  if (domega_bias) P.seg[P.nseg++] = PartSeg{part_bias, (int64_t)2 * H, H, domega_bias};
  if (dr_bias) P.seg[P.nseg++] = PartSeg{part_bias + H, (int64_t)2 * H, H, dr_bias};
  P.mu_param = mu_param;
  P.H = H;
  P.dmu_param = dmu_param;  // the gain's prior is mu only without an initial precision (else zero)
  if (prec_mode == 0 && rows) {
    P.dmu_rows = rows;
    P.nrows = B;
    P.rows_to_param = initial_precision ? 0 : 1;
    P.dmu_sum = initial_precision ? d_initial_precision : nullptr;
  }
  const int nblk = part_segs_blocks(P);
  if (nblk > 0) hipLaunchKernelGGL(reduce_partials_multi_kernel, dim3(nblk), dim3(256), 0, stream, P, NP);
  KDN_CHECK_LAUNCH();
  return 0;
}

int kdn_l2norm_fwd(const void* x, int x_bf16, int64_t rows, int K, float eps, void* y, int y_bf16, float* rstd,
                   hipStream_t stream) {
  if (K <= 0 || K > 256 || rows < 0) return KDN_ERR_ARG;
  if (rows == 0) return 0;
  if (row_vec_ok(K) && aligned16(x) && aligned16(y)) {
    dim3 gv(cdiv(rows, 256 / (K / 8)));
#define KDN_L2F(TX, TY)                                                                                            \
  hipLaunchKernelGGL((l2norm_fwd_vec_kernel<TX, TY>), gv, dim3(256), 0, stream, (const TX*)x, rows, K, eps, (TY*)y, \
                     rstd)
    if (x_bf16 && y_bf16) KDN_L2F(bf16_t, bf16_t);
    else if (x_bf16) KDN_L2F(bf16_t, float);
    else if (y_bf16) KDN_L2F(float, bf16_t);
    else KDN_L2F(float, float);
#undef KDN_L2F
    KDN_CHECK_LAUNCH();
    return 0;
  }
  dim3 grid(cdiv(rows, 4));
  if (x_bf16 && y_bf16)
    hipLaunchKernelGGL((l2norm_fwd_kernel<bf16_t, bf16_t>), grid, dim3(256), 0, stream, (const bf16_t*)x, rows, K, eps, (bf16_t*)y, rstd);
  else if (x_bf16)
    hipLaunchKernelGGL((l2norm_fwd_kernel<bf16_t, float>), grid, dim3(256), 0, stream, (const bf16_t*)x, rows, K, eps, (float*)y, rstd);
  else if (y_bf16)
    hipLaunchKernelGGL((l2norm_fwd_kernel<float, bf16_t>), grid, dim3(256), 0, stream, (const float*)x, rows, K, eps, (bf16_t*)y, rstd);
  else
    hipLaunchKernelGGL((l2norm_fwd_kernel<float, float>), grid, dim3(256), 0, stream, (const float*)x, rows, K, eps, (float*)y, rstd);
  KDN_CHECK_LAUNCH();
  return 0;
}

int kdn_l2norm_bwd(const void* x, int x_bf16, const float* rstd, const void* dy, int dy_bf16, int64_t rows, int K,
                   void* dx, hipStream_t stream) {
  if (K <= 0 || K > 256 || rows < 0) return KDN_ERR_ARG;
  if (rows == 0) return 0;
  if (row_vec_ok(K) && aligned16(x) && aligned16(dy) && aligned16(dx)) {
    dim3 gv(cdiv(rows, 256 / (K / 8)));
#define KDN_L2B(TX, TD)                                                                                           \
  hipLaunchKernelGGL((l2norm_bwd_vec_kernel<TX, TD>), gv, dim3(256), 0, stream, (const TX*)x, rstd, (const TD*)dy, \
                     rows, K, (TX*)dx)
    if (x_bf16 && dy_bf16) KDN_L2B(bf16_t, bf16_t);
    else if (x_bf16) KDN_L2B(bf16_t, float);
    else if (dy_bf16) KDN_L2B(float, bf16_t);
    else KDN_L2B(float, float);
#undef KDN_L2B
    KDN_CHECK_LAUNCH();
    return 0;
  }
  dim3 grid(cdiv(rows, 4));
  if (x_bf16 && dy_bf16)
    hipLaunchKernelGGL((l2norm_bwd_kernel<bf16_t, bf16_t>), grid, dim3(256), 0, stream, (const bf16_t*)x, rstd, (const bf16_t*)dy, rows, K, (bf16_t*)dx);
  else if (x_bf16)
    hipLaunchKernelGGL((l2norm_bwd_kernel<bf16_t, float>), grid, dim3(256), 0, stream, (const bf16_t*)x, rstd, (const float*)dy, rows, K, (bf16_t*)dx);
  else if (dy_bf16)
    hipLaunchKernelGGL((l2norm_bwd_kernel<float, bf16_t>), grid, dim3(256), 0, stream, (const float*)x, rstd, (const bf16_t*)dy, rows, K, (float*)dx);
  else
    hipLaunchKernelGGL((l2norm_bwd_kernel<float, float>), grid, dim3(256), 0, stream, (const float*)x, rstd, (const float*)dy, rows, K, (float*)dx);
  KDN_CHECK_LAUNCH();
  return 0;
}

int kdn_diag_norm_fwd(const void* q_raw, const void* k_raw, int x_bf16, int64_t rows, int K, uint16_t* q_memory,
                      float* k_gain, uint16_t* k_memory, float* q_norm, float* k_norm, hipStream_t stream) {
  if (K <= 0 || K > 256 || rows < 0) return KDN_ERR_ARG;
  if (rows == 0) return 0;
  if (row_vec_ok(K) && aligned16(q_raw) && aligned16(k_raw) && aligned16(q_memory) && aligned16(k_gain) &&
      aligned16(k_memory)) {
    dim3 gv(cdiv(rows, 256 / (K / 8)));
    if (x_bf16)
      hipLaunchKernelGGL((diag_norm_fwd_vec_kernel<bf16_t>), gv, dim3(256), 0, stream, (const bf16_t*)q_raw,
                         (const bf16_t*)k_raw, rows, K, q_memory, k_gain, k_memory, q_norm, k_norm);
    else
      hipLaunchKernelGGL((diag_norm_fwd_vec_kernel<float>), gv, dim3(256), 0, stream, (const float*)q_raw,
                         (const float*)k_raw, rows, K, q_memory, k_gain, k_memory, q_norm, k_norm);
    KDN_CHECK_LAUNCH();
    return 0;
  }
  dim3 grid(cdiv(rows, 4));
  if (x_bf16)
    hipLaunchKernelGGL((diag_norm_fwd_kernel<bf16_t>), grid, dim3(256), 0, stream, (const bf16_t*)q_raw, (const bf16_t*)k_raw, rows, K, q_memory, k_gain, k_memory, q_norm, k_norm);
  else
    hipLaunchKernelGGL((diag_norm_fwd_kernel<float>), grid, dim3(256), 0, stream, (const float*)q_raw, (const float*)k_raw, rows, K, q_memory, k_gain, k_memory, q_norm, k_norm);
  KDN_CHECK_LAUNCH();
  return 0;
}

int kdn_diag_norm_bwd(const void* q_raw, const void* k_raw, int x_bf16, const float* q_norm, const float* k_norm,
                      const uint16_t* d_q_memory, const float* d_k_gain, const uint16_t* d_k_memory, int64_t rows,
                      int K, void* dq_raw, void* dk_raw, hipStream_t stream) {
  if (K <= 0 || K > 256 || rows < 0) return KDN_ERR_ARG;
  if (rows == 0) return 0;
  if (row_vec_ok(K) && aligned16(q_raw) && aligned16(k_raw) && aligned16(d_q_memory) && aligned16(d_k_gain) &&
      aligned16(d_k_memory) && aligned16(dq_raw) && aligned16(dk_raw)) {
    dim3 gv(cdiv(rows, 256 / (K / 8)));
    if (x_bf16)
      hipLaunchKernelGGL((diag_norm_bwd_vec_kernel<bf16_t>), gv, dim3(256), 0, stream, (const bf16_t*)q_raw,
                         (const bf16_t*)k_raw, q_norm, k_norm, d_q_memory, d_k_gain, d_k_memory, rows, K,
                         (bf16_t*)dq_raw, (bf16_t*)dk_raw);
    else
      hipLaunchKernelGGL((diag_norm_bwd_vec_kernel<float>), gv, dim3(256), 0, stream, (const float*)q_raw,
                         (const float*)k_raw, q_norm, k_norm, d_q_memory, d_k_gain, d_k_memory, rows, K,
                         (float*)dq_raw, (float*)dk_raw);
    KDN_CHECK_LAUNCH();
    return 0;
  }
  dim3 grid(cdiv(rows, 4));
  if (x_bf16)
    hipLaunchKernelGGL((diag_norm_bwd_kernel<bf16_t>), grid, dim3(256), 0, stream, (const bf16_t*)q_raw, (const bf16_t*)k_raw, q_norm, k_norm, d_q_memory, d_k_gain, d_k_memory, rows, K, (bf16_t*)dq_raw, (bf16_t*)dk_raw);
  else
    hipLaunchKernelGGL((diag_norm_bwd_kernel<float>), grid, dim3(256), 0, stream, (const float*)q_raw, (const float*)k_raw, q_norm, k_norm, d_q_memory, d_k_gain, d_k_memory, rows, K, (float*)dq_raw, (float*)dk_raw);
  KDN_CHECK_LAUNCH();
  return 0;
}

int kdn_diag_frontend_fwd(const uint16_t* retention_raw, const uint16_t* omega_raw, const uint16_t* r_raw,
                          const float* A_log, const float* dt_bias, const float* mu_param, int B, int T, int H, int K,
                          int chunk, float* g_cumsum, float* alpha, float* omega, float* r, float* mu,
                          hipStream_t stream) {
  if (K <= 0 || K > 256 || chunk <= 0 || B <= 0 || T <= 0 || H <= 0) return KDN_ERR_ARG;
  const int NT = cdiv(T, chunk);
  const bool vec = gate_vec_ok(K, chunk) && aligned16(retention_raw) && aligned16(omega_raw) && aligned16(dt_bias) &&
                   aligned16(g_cumsum) && aligned16(alpha) && aligned16(omega);
  hipLaunchKernelGGL(vec ? diag_frontend_fwd_vec_kernel : diag_frontend_fwd_kernel, dim3(H * B * NT), dim3(256), 0,
                     stream, retention_raw, omega_raw, r_raw, A_log, dt_bias, mu_param, T, H, K, chunk, NT, g_cumsum,
                     alpha, omega, r, mu);
  KDN_CHECK_LAUNCH();
  return 0;
}

size_t kdn_diag_frontend_bwd_workspace_size(int B, int T, int H, int K, int chunk) {
  const int64_t NP = (int64_t)B * cdiv(T, chunk);
  return (size_t)(NP * H + NP * H * K) * sizeof(float);
}

int kdn_diag_frontend_bwd(const uint16_t* retention_raw, const uint16_t* omega_raw, const uint16_t* r_raw,
                          const float* A_log, const float* dt_bias, const float* mu_param, const float* alpha,
                          const float* d_g_cumsum, const float* d_alpha, const float* d_omega, const float* d_r,
                          const float* d_mu, int B, int T, int H, int K, int chunk, uint16_t* d_retention_raw,
                          uint16_t* d_omega_raw, uint16_t* d_r_raw, float* dA_log, float* ddt_bias,
                          float* d_mu_param, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (K <= 0 || K > 256 || chunk <= 0 || B <= 0 || T <= 0 || H <= 0) return KDN_ERR_ARG;
  if (workspace_bytes < kdn_diag_frontend_bwd_workspace_size(B, T, H, K, chunk)) return KDN_ERR_ARG;
  const int NT = cdiv(T, chunk);
  const int NP = B * NT;
  float* part_A = (float*)workspace;
  float* part_dt = part_A + (int64_t)NP * H;
  const bool has_decay = d_g_cumsum || d_alpha;
  if (has_decay && (d_retention_raw || dA_log || ddt_bias)) {
    const bool vec = gate_vec_ok(K, chunk) && aligned16(retention_raw) && aligned16(dt_bias) && aligned16(alpha) &&
                     aligned16(d_g_cumsum) && aligned16(d_alpha) && aligned16(d_retention_raw);
    hipLaunchKernelGGL(vec ? diag_frontend_bwd_vec_kernel : diag_frontend_bwd_kernel, dim3(H * NP), dim3(256), 0,
                       stream, retention_raw, A_log, dt_bias, alpha, d_g_cumsum, d_alpha, T, H, K, chunk, NT,
                       d_retention_raw, dA_log ? part_A : nullptr, ddt_bias ? part_dt : nullptr);
    KDN_CHECK_LAUNCH();
    if (dA_log)
      hipLaunchKernelGGL(reduce_partials_vec_kernel, dim3(cdiv(H, 64)), dim3(256), 0, stream, part_A, NP, (int64_t)H, H,
                         dA_log);
    if (ddt_bias)
      hipLaunchKernelGGL(reduce_partials_vec_kernel, dim3(cdiv(H * K, 64)), dim3(256), 0, stream, part_dt, NP,
                         (int64_t)H * K, H * K, ddt_bias);
  } else {
    const int64_t n = (int64_t)B * T * H * K;
    if (d_retention_raw) hipLaunchKernelGGL(fill_zero_kernel<uint16_t>, dim3(cdiv(n, 256)), dim3(256), 0, stream, d_retention_raw, n);
    if (dA_log) hipLaunchKernelGGL(fill_zero_kernel<float>, dim3(cdiv(H, 256)), dim3(256), 0, stream, dA_log, (int64_t)H);
    if (ddt_bias) hipLaunchKernelGGL(fill_zero_kernel<float>, dim3(cdiv((int64_t)H * K, 256)), dim3(256), 0, stream, ddt_bias, (int64_t)H * K);
  }
  if (d_omega_raw && d_omega) {
    const int64_t n = (int64_t)B * T * H * K;
    hipLaunchKernelGGL(sigmoid_vjp_kernel, dim3(cdiv(n, 256)), dim3(256), 0, stream, omega_raw, d_omega, n, d_omega_raw);
  }
  if (d_r_raw && d_r) {
    const int64_t n = (int64_t)B * T * H;
    hipLaunchKernelGGL(sigmoid_vjp_kernel, dim3(cdiv(n, 256)), dim3(256), 0, stream, r_raw, d_r, n, d_r_raw);
  }
  if (d_mu_param) hipLaunchKernelGGL(mu_vjp_kernel, dim3(cdiv(H, 256)), dim3(256), 0, stream, mu_param, d_mu, H, d_mu_param);
  KDN_CHECK_LAUNCH();
  return 0;
}

}  // extern "C"
