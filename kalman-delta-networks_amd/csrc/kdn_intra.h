// Forward intra-chunk kernels of the KDN memory scan, MFMA formulation.
//
// Per chunk (C = 64 tokens) with G the base-2 chunk-local prefix of the log gate:
//   N[c,s] = sum_i k_ci kappa_si 2^{G_ci - G_si} (s < c),  M[c,s] = scale sum_i q_ci kappa_si 2^{G_ci - G_si} (s <= c)
//   A = (I + N)^{-1}:  16x16 diagonal blocks by substitution, off-diagonal blocks level by level
//                      A_IJ = -A_II sum_{J<=P<I} N_IP A_PJ           (fp32 MFMA)
//   U = A V,  W = A (k 2^G),  Kf = kappa 2^{G_last - G},  Qg = scale q 2^G
// N and M are K-contractions of factored operands (bf16x3 MFMA); the decay 2^{G_c - G_s} is split
// at an anchor so neither factor overflows.  A^T is saved for the backward.
//
// intra_fwd_kernel (every chunk): one anchor per chunk and channel, the midpoint of the chunk's gate
//   range m = (G_0 + G_{L-1}) / 2, so |G - m| <= span / 2 on every row:
//   Lk = k 2^{G - m},  Lq = scale q 2^{G - m},  R = kappa 2^{m - G}  (each <= 2^{span/2} times k, q, kappa);
//   a chunk whose span max_i (G_0 - G_{L-1})_i exceeds kAnchorSpanMax is flagged (flags = 1).
// intra_fwd_block_chunk (each flagged chunk, in one launch with the exact path): one anchor per 16-token block J,
//   m_J = (G_{16J} + G_{16J+15})/2 per channel (rows clamped), so |G - m_J| <= span_J / 2 inside
//   the block.  For s in block J and c in block I >= J, 2^{G_c - G_s} = (2^{G_c - m_J}) (2^{m_J - G_s}):
//   R_J = kappa 2^{m_J - G} (published per block),  Lk_IJ = k 2^{G - m_I} 2^{m_I - m_J}  (<= 1 for J < I),
//   Lq likewise.  A chunk handled here gets flags = 0; one with a block span past kBlockSpanMax
//   (the masked upper-triangle products of a diagonal block reach 2^span) stays flagged for the
//   exact per-block path, which the same workgroup then runs.
// A random-init 1.3B model decays by up to ~e^-2 per token in its fastest channels on average (chunk
// spans up to ~170), which the midpoint anchor covers; faster decay (trained models reach ~e^-4 per
// token, spans ~370) takes the block kernel.
//
// Layout of work: wave w owns row block I = w (16 rows) for the N / M build, keeping its k / q
// factors in registers and publishing its R fragments (and block anchors) to LDS; the U / W
// products are split over the waves by output column tile.
#pragma once
#include <type_traits>
#include "kdn_common.h"
#include "kdn_state.h"

namespace kdn_intra {

using kdn_state::afrag;
using kdn_state::bfrag;
using kdn_state::C;
using kdn_state::mfma;
using kdn_state::mma2;
using kdn_state::mma3;
using kdn_state::wave_lds_sync;
using kdn_state::split2;
using kdn_state::TILE;
using kdn_state::zero4;

// base 2, one midpoint anchor per chunk and channel: every factor stays <= 2^100, far inside fp32 (the
// masked products above the diagonal may overflow; they are discarded by a select, never multiplied)
constexpr float kAnchorSpanMax = 200.f;
constexpr float kBlockSpanMax = 120.f;   // base 2, per 16-token block: every product stays below 2^120
constexpr int AP = C + 1;                // LDS row stride of the fp32 N and A tiles
constexpr int XR = 128 + 4;              // LDS row stride of the staged [s][column] operands (<= 128 columns)

__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
// 8 bf16 (raw bits in a uint4) -> 8 floats
__device__ __forceinline__ void unpack8(u32x4 v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    f[2 * p] = __uint_as_float(w[p] << 16);
    f[2 * p + 1] = __uint_as_float(w[p] & 0xffff0000u);
  }
}
__device__ __forceinline__ void split8(const float* x, uint4& hi, uint4& lo) {
  split2(x[0], x[1], hi.x, lo.x);
  split2(x[2], x[3], hi.y, lo.y);
  split2(x[4], x[5], hi.z, lo.z);
  split2(x[6], x[7], hi.w, lo.w);
}
// (hi + lo) * f, re-split: the split pair holds the value to 2^-17 relative
__device__ __forceinline__ void rescale8(const uint4& hi, const uint4& lo, const float* f, uint4& oh, uint4& ol) {
  const uint32_t h[4] = {hi.x, hi.y, hi.z, hi.w}, l[4] = {lo.x, lo.y, lo.z, lo.w};
  float x[8];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    x[2 * p] = (__uint_as_float(h[p] << 16) + __uint_as_float(l[p] << 16)) * f[2 * p];
    x[2 * p + 1] = (__uint_as_float(h[p] & 0xffff0000u) + __uint_as_float(l[p] & 0xffff0000u)) * f[2 * p + 1];
  }
  split8(x, oh, ol);
}
__device__ __forceinline__ void ld8(bufrsrc r, uint32_t off, float* f) {
  const float4 a = buf_ld4(r, off), b = buf_ld4(r, off + 16);
  f[0] = a.x, f[1] = a.y, f[2] = a.z, f[3] = a.w, f[4] = b.x, f[5] = b.y, f[6] = b.z, f[7] = b.w;
}
__device__ __forceinline__ void st8(bufrsrc r, uint32_t off, const float* f) {
  __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                                               __float_as_uint(f[3])},
                                         r, off, 0, 0);
  __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(f[4]), __float_as_uint(f[5]), __float_as_uint(f[6]),
                                               __float_as_uint(f[7])},
                                         r, off + 16, 0, 0);
}

// Stages after the N / M build, shared by both kernels: the inverse A = (I + N)^{-1} from sN, A^T
// saved to An, then U = A V and W = A (k 2^G) (rows past L dropped by the output descriptors).
// The whole LDS buffer (sA / sN / sX) is free for this function's staging after the first barrier.
// NORM (in-op L2 norm): k is raw in memory, sRk holds the rows' rstd.
template <int K, int V, bool NORM>
__device__ __forceinline__ void intra_solve_emit(float* sA, float* sN, float* sX, float* An, bufrsrc rv, bufrsrc rk,
                                                 bufrsrc rG, bufrsrc rU, bufrsrc rW, int H, int tid,
                                                 const float* sRk) {
  const int lane = tid & 63, w = tid >> 6, r16 = lane & 15, g4 = lane >> 4;
  // ---- 3. diagonal blocks of A: X_I = (I + N_II)^{-1}, lane j < 16 of wave I owns column j
  if (lane < 16) {
    const int base = 16 * w, j = lane;
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = r == j ? 1.f : 0.f;
#pragma unroll
    for (int r = 1; r < 16; ++r) {
      float acc = 0.f;
#pragma unroll
      for (int m = 0; m < r; ++m) acc -= sN[(base + r) * AP + base + m] * x[m];
      if (r > j) x[r] = acc;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) sA[(base + r) * AP + base + j] = x[r];
  }
  // blocks above the diagonal are zero
  for (int e = lane; e < 256 * (3 - w); e += 64) {
    const int J = w + 1 + (e >> 8), rr = (e >> 4) & 15, cc = e & 15;
    sA[(16 * w + rr) * AP + 16 * J + cc] = 0.f;
  }
  __syncthreads();

  // ---- 4. off-diagonal blocks, one block-row level at a time: wave J makes A_IJ
#pragma unroll
  for (int I = 1; I < 4; ++I) {
    if (w < I) {
      const int J = w;
      f32x4 t = zero4();
      for (int P = J; P < I; ++P) {
#pragma unroll
        for (int st = 0; st < 4; ++st)
          t = mfma_f32(sN[(16 * I + r16) * AP + 16 * P + 4 * st + g4], sA[(16 * P + 4 * st + g4) * AP + 16 * J + r16],
                       t);
      }
      // A_IJ = -X_I T; the k index of step st is 4 g4 + st, so T comes straight from the D layout
      f32x4 o = zero4();
#pragma unroll
      for (int st = 0; st < 4; ++st) o = mfma_f32(sA[(16 * I + r16) * AP + 16 * I + 4 * g4 + st], t[st], o);
#pragma unroll
      for (int j = 0; j < 4; ++j) sA[(16 * I + 4 * g4 + j) * AP + 16 * J + r16] = -o[j];
    }
    __syncthreads();
  }

  // ---- 5. save A^T ([s][c], the orientation the backward contracts over) for the backward
  {
    const bufrsrc rA = make_buf(An, An ? C * C * 4 : 0u);  // no backward follows: nothing to save
#pragma unroll
    for (int u = 0; u < C * C / 4 / 256; ++u) {
      const int e = 4 * (tid + 256 * u), sr = e / C, c0 = e % C;  // A^T[sr][c0 .. c0+3] = A[c0 + j][sr]
      const float4 x = float4{sA[c0 * AP + sr], sA[(c0 + 1) * AP + sr], sA[(c0 + 2) * AP + sr], sA[(c0 + 3) * AP + sr]};
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), rA, e * 4, 0, 0);
    }
  }

  // ---- 6. U = A V, W = A (k 2^G) over output column tiles t (V/16 of U, then K/16 of W)
  // A fragments in the permuted k order of the accumulator-layout B operands:
  // slots 0-3 <- s = 32 kb + 4 g4 + (0..3), slots 4-7 <- s = 32 kb + 16 + 4 g4 + (0..3)
  uint4 ah[4][2], al[4][2];
#pragma unroll
  for (int I = 0; I < 4; ++I)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      if (kb == 1 && I < 2) continue;
      const float* row = sA + (16 * I + r16) * AP + 32 * kb + 4 * g4;
      const float x[8] = {row[0], row[1], row[2], row[3], row[16], row[17], row[18], row[19]};
      split8(x, ah[I][kb], al[I][kb]);
    }
  // U = A V and W = A Kg (Kg = k 2^G) in transposed form: the operand (loaded coalesced as rows and
  // staged in LDS row-major [s][col], read back by columns) is the A fragment and A's rows the B fragment, so the D
  // tile gives each lane 4 consecutive output columns of one chunk row (16-byte stores).
  __syncthreads();  // every wave has its A fragments; the buffer is free
  auto stage = [&](auto is_u) {
    constexpr bool isU = decltype(is_u)::value;
    constexpr int D = isU ? V : K, UNITS = C * D / 8 / 256;
#pragma unroll
    for (int u = 0; u < UNITS; ++u) {
      const int e = tid + 256 * u, sr = e / (D / 8), c8 = 8 * (e % (D / 8));
      const uint32_t o = (uint32_t)(sr * H) * D + c8;
      float x[8];
      if constexpr (isU) {
        unpack8(__builtin_amdgcn_raw_buffer_load_b128(rv, o * 2, 0, 0), x);
      } else {
        float g[8];
        unpack8(__builtin_amdgcn_raw_buffer_load_b128(rk, o * 2, 0, 0), x);
        ld8(rG, o * 4, g);
        if constexpr (NORM) {
          const float rs = sRk[sr];
#pragma unroll
          for (int j = 0; j < 8; ++j) x[j] = l2n(x[j], rs);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] *= fexp2(g[j]);
      }
      // row-major [s][col]: the 16 lanes of a row write consecutive 16-byte pieces (a column-major
      // store here put 16 lanes on one bank)
      *reinterpret_cast<float4*>(sX + sr * XR + c8) = float4{x[0], x[1], x[2], x[3]};
      *reinterpret_cast<float4*>(sX + sr * XR + c8 + 4) = float4{x[4], x[5], x[6], x[7]};
    }
  };
  auto tile = [&](auto is_u, int t) {
    constexpr bool isU = decltype(is_u)::value;
    constexpr int D = isU ? V : K;
    uint4 xh[2], xl[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      // column 16 t + r16, rows 32 kb + 4 g4 + (0..3) and + 16: with the row pitch XR = 4 (mod 64)
      // the 64 lanes of each read fall on 64 different banks
      const float* colp = sX + (32 * kb + 4 * g4) * XR + 16 * t + r16;
      float x[8];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        x[jj] = colp[jj * XR];
        x[4 + jj] = colp[(16 + jj) * XR];
      }
      split8(x, xh[kb], xl[kb]);  // exact for V (lo = 0)
    }
    const bufrsrc rO = isU ? rU : rW;
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      f32x4 acc = zero4();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        if (kb == 1 && I < 2) continue;  // A[c][s] = 0 for s > c
        acc = mfma(xh[kb], ah[I][kb], acc);
        acc = mfma(xh[kb], al[I][kb], acc);
        if constexpr (!isU) acc = mfma(xl[kb], ah[I][kb], acc);
      }
      const uint32_t row = (uint32_t)(16 * I + r16);  // rows past L are dropped by the descriptor
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc), rO,
                                             (row * D + 16 * t + 4 * g4) * 4, 0, 0);
    }
  };
  stage(std::true_type{});
  __syncthreads();
  for (int t = w; t < V / 16; t += 4) tile(std::true_type{}, t);
  __syncthreads();
  stage(std::false_type{});
  __syncthreads();
  for (int t = w; t < K / 16; t += 4) tile(std::false_type{}, t);
}

// In-op L2 norm of a chunk row held by the four lane groups of a wave (lane group g4 = lane >> 4
// holds channels 32 kb + 8 g4 .. + 7 as raw bf16): the row's rstd, its sum of squares taken in the
// order of l2norm_fwd_vec_kernel (runs of 8 channels, then the xor tree: g4 ^ 1, g4 ^ 2 across lanes,
// kb pairs in the lane), so it is bit-identical to that kernel's.
template <int KB>
__device__ __forceinline__ float row_rstd(const u32x4 (&raw)[KB]) {
  float t[KB];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    float x[8];
    unpack8(raw[kb], x);
    t[kb] = l2n_run(x);
  }
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) t[kb] = t[kb] + __shfl_xor(t[kb], 16, 64);
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) t[kb] = t[kb] + __shfl_xor(t[kb], 32, 64);
  return l2n_rstd(l2n_tree<KB>(t));
}

// grid (chunks, B*H), block 256: chunks n0 .. n0 + gridDim.x - 1 of every head.
template <int K, int V, bool ISO, bool NORM = false>
__global__ __launch_bounds__(256, 3) void intra_fwd_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const float* __restrict__ kap,
    const bf16_t* __restrict__ v, const float* __restrict__ gc, int T, int H, int NT, float scale,
    float* __restrict__ U, float* __restrict__ W, float* __restrict__ Kf, float* __restrict__ Qg,
    float* __restrict__ Mg, float* __restrict__ Ag, int* __restrict__ flags, float* __restrict__ q_rstd = nullptr,
    float* __restrict__ k_rstd = nullptr, int n0 = 0) {
  constexpr int KB = K / 32;
  // R fragments [s-tile][kb] until the N / M build, then A [c][s] in the same bytes
  constexpr int RBYTES = (C / 16) * KB * TILE * 2, ABYTES = C * AP * 4;
  constexpr int RABYTES = RBYTES > ABYTES ? RBYTES : ABYTES;
  // [R fragments | A] then N [c][s]; the U/W stage reuses the whole buffer for its operand staging
  constexpr int SBYTES = RABYTES + C * AP * 4 > C * XR * 4 ? RABYTES + C * AP * 4 : C * XR * 4;
  static_assert(V <= 128 && K <= 128, "operand staging holds up to 128 columns");
  __shared__ __attribute__((aligned(16))) unsigned char sbuf[SBYTES];
  __shared__ float sRk[C];  // in-op L2 norm: the rows' k rstd for the W stage
  bf16_t* sR = reinterpret_cast<bf16_t*>(sbuf);
  float* sA = reinterpret_cast<float*>(sbuf);
  float* sN = reinterpret_cast<float*>(sbuf + RABYTES);
  float* sX = reinterpret_cast<float*>(sbuf);  // U/W stage: operand rows [s][col], pitch XR
  const int n = n0 + blockIdx.x, bh = blockIdx.y, b = bh / H, h = bh % H;  // chunks n0 + gridDim.x
  const int t0 = n * C, L = min(C, T - t0);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r16 = lane & 15, g4 = lane >> 4;

  // [B,T,H,D] inputs: row c of this chunk at ((b*T + t0 + c)*H + h)*D
  const int64_t in_row0 = ((int64_t)b * T + t0) * H + h;
  const uint32_t rows_in = (uint32_t)((L - 1) * H + 1);  // descriptor covers rows 0..L-1 of this head
  const bufrsrc rG = make_buf(gc + in_row0 * K, rows_in * K * 4);
  const bufrsrc rk = make_buf(k + in_row0 * K, rows_in * K * 2);
  const bufrsrc rq = make_buf(q + in_row0 * K, rows_in * K * 2);
  const bufrsrc rkap = ISO ? make_buf(kap + in_row0, rows_in * 4) : make_buf(kap + in_row0 * K, rows_in * K * 4);
  const bufrsrc rv = make_buf(v + in_row0 * V, rows_in * V * 2);
  // [B*H, T, D] outputs
  const bufrsrc rKf = make_buf(Kf + ((int64_t)bh * T + t0) * K, L * K * 4);
  const bufrsrc rQg = make_buf(Qg + ((int64_t)bh * T + t0) * K, L * K * 4);
  const bufrsrc rU = make_buf(U + ((int64_t)bh * T + t0) * V, L * V * 4);
  const bufrsrc rW = make_buf(W + ((int64_t)bh * T + t0) * K, L * K * 4);
  float* Mn = Mg + ((int64_t)bh * NT + n) * C * C;
  float* An = Ag ? Ag + ((int64_t)bh * NT + n) * C * C : nullptr;

  // ---- 0. the chunk's decay span max_i (G_0 - G_{L-1})_i, from rows 0 and L-1 alone, before any
  // other load or store: a chunk past the single anchor's range goes to the block-anchor kernel
  // without paying for the rest.  Lane groups g4 cover all K channels, so every wave computes the
  // same span and the early return is uniform across the workgroup (no barrier needed).
  float g0s[KB][8], gls[KB][8];  // rows 0 and L-1, kept for stage 1
  {
    float span = 0.f;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int i0 = 32 * kb + 8 * g4;
      ld8(rG, i0 * 4, g0s[kb]);
      ld8(rG, ((uint32_t)((L - 1) * H) * K + i0) * 4, gls[kb]);
#pragma unroll
      for (int j = 0; j < 8; ++j) span = fmaxf(span, g0s[kb][j] - gls[kb][j]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) span = fmaxf(span, __shfl_xor(span, o, 64));
    if (!(span <= kAnchorSpanMax)) {  // the block-anchor kernel (or, past it, the exact one) takes this chunk
      if (tid == 0) flags[(int64_t)bh * NT + n] = 1;
      return;
    }
  }
  if (tid == 0) flags[(int64_t)bh * NT + n] = 0;

  // ---- 1. per-row factors: wave w owns rows 16w + r16; lanes hold 8 consecutive channels.
  // Rows past L read zero k, q, kappa and repeat the gate of row L-1, so every factor is bounded.
  const int c = 16 * w + r16;
  const uint32_t crow = (uint32_t)(c * H), grow = (uint32_t)(min(c, L - 1) * H);
  uint4 lkh[KB], lkl[KB], lqh[KB], lql[KB];
  const float beta = ISO ? buf_ld(rkap, crow * 4) : 0.f;
  // Kf and Qg leave through this wave's slice of the N tile's bytes (unused until stage 2): a lane's 8
  // channels lie 32 bytes from the next lane's, so a direct store covers 16 rows in 16-byte pieces;
  // regrouped, each store writes 8 whole 128-byte row segments.  Slice: [Kf | Qg][16 rows][32 channels],
  // 16-byte quad q of row r at slot q ^ (r & 7).
  static_assert(4 * 2 * 16 * 32 * 4 <= C * AP * 4, "Kf / Qg staging fits the N tile");
  float* sKQ = sN + w * (2 * 16 * 32);
  // with the in-op L2 norm (NORM) q, k are raw: this workgroup normalises its rows
  float rsq = 1.f, rsk = 1.f;
  u32x4 kraw[KB], qraw[KB];
  if constexpr (NORM) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      kraw[kb] = __builtin_amdgcn_raw_buffer_load_b128(rk, (crow * K + 32 * kb + 8 * g4) * 2, 0, 0);
      qraw[kb] = __builtin_amdgcn_raw_buffer_load_b128(rq, (crow * K + 32 * kb + 8 * g4) * 2, 0, 0);
    }
    rsq = row_rstd<KB>(qraw);
    rsk = row_rstd<KB>(kraw);
    if (g4 == 0) {
      buf_st(make_buf(q_rstd + in_row0, rows_in * 4), crow * 4, rsq);  // rows past L are dropped
      buf_st(make_buf(k_rstd + in_row0, rows_in * 4), crow * 4, rsk);
      sRk[c] = rsk;
    }
  }
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const int i0 = 32 * kb + 8 * g4;
    float gcv[8], kv[8], qv[8], av[8];
    float g0x[8], glx[8];
    if constexpr (NORM) {  // rows 0 and L-1 again (cached): the raw q, k rows take their registers
      ld8(rG, i0 * 4, g0x);
      ld8(rG, ((uint32_t)((L - 1) * H) * K + i0) * 4, glx);
    }
    const float* g0 = NORM ? g0x : g0s[kb];
    const float* gl = NORM ? glx : gls[kb];
    ld8(rG, (grow * K + i0) * 4, gcv);
    if constexpr (NORM) {
      unpack8(kraw[kb], kv);
      unpack8(qraw[kb], qv);
    } else {
      unpack8(__builtin_amdgcn_raw_buffer_load_b128(rk, (crow * K + i0) * 2, 0, 0), kv);
      unpack8(__builtin_amdgcn_raw_buffer_load_b128(rq, (crow * K + i0) * 2, 0, 0), qv);
    }
    if constexpr (NORM) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        kv[j] = l2n(kv[j], rsk);
        qv[j] = l2n(qv[j], rsq);
      }
    }
    if (ISO) {
#pragma unroll
      for (int j = 0; j < 8; ++j) av[j] = beta * kv[j];
    } else {
      ld8(rkap, (crow * K + i0) * 4, av);
    }
    float lk[8], lq[8], rr[8], kf[8], qg[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float mid = 0.5f * (g0[j] + gl[j]);
      const float e = fexp2(gcv[j] - mid);
      lk[j] = kv[j] * e;
      lq[j] = scale * qv[j] * e;
      rr[j] = av[j] * fexp2(mid - gcv[j]);
      kf[j] = av[j] * fexp2(gl[j] - gcv[j]);
      qg[j] = scale * qv[j] * fexp2(gcv[j]);
    }
    split8(lk, lkh[kb], lkl[kb]);
    split8(lq, lqh[kb], lql[kb]);
    uint4 rh, rl;
    split8(rr, rh, rl);
    *reinterpret_cast<uint4*>(sR + (w * KB + kb) * TILE + lane * 8) = rh;
    *reinterpret_cast<uint4*>(sR + (w * KB + kb) * TILE + 512 + lane * 8) = rl;
    wave_lds_sync();  // the previous column block's reads are issued before these writes
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      float* slot = sKQ + r16 * 32 + (((2 * g4 + hf) ^ (r16 & 7)) * 4);
      *reinterpret_cast<float4*>(slot) = float4{kf[4 * hf], kf[4 * hf + 1], kf[4 * hf + 2], kf[4 * hf + 3]};
      *reinterpret_cast<float4*>(slot + 512) = float4{qg[4 * hf], qg[4 * hf + 1], qg[4 * hf + 2], qg[4 * hf + 3]};
    }
    wave_lds_sync();
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int rr = (lane >> 3) + 8 * hh, qd = lane & 7;
      const float* slot = sKQ + rr * 32 + ((qd ^ (rr & 7)) * 4);
      const uint32_t off = ((uint32_t)(16 * w + rr) * K + 32 * kb + 4 * qd) * 4;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, *reinterpret_cast<const float4*>(slot)),
                                             rKf, off, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b128(
          __builtin_bit_cast(u32x4, *reinterpret_cast<const float4*>(slot + 512)), rQg, off, 0, 0);
    }
  }
  __syncthreads();  // R fragments of every row block; the N tile's bytes are free again

  // ---- 2. N and M tiles of row block I = w
  const bufrsrc rM = make_buf(Mn, C * C * 4);
#pragma unroll
  for (int J = 0; J < 4; ++J) {
    const int s = 16 * J + r16;
    if (J <= w) {
      f32x4 aN = zero4(), aM = zero4();
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        uint4 rh, rl;
        afrag(sR, J * KB + kb, lane, rh, rl);
        aN = mma3(lkh[kb], lkl[kb], rh, rl, aN);
        aM = mma3(lqh[kb], lql[kb], rh, rl, aM);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int cc = 16 * w + 4 * g4 + j;
        sN[cc * AP + s] = (J < w || s < cc) ? aN[j] : 0.f;
        buf_st(rM, (cc * C + s) * 4, (J < w || s <= cc) ? aM[j] : 0.f);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) buf_st(rM, ((16 * w + 4 * g4 + j) * C + s) * 4, 0.f);
    }
  }
  __syncthreads();

  intra_solve_emit<K, V, NORM>(sA, sN, sX, An, rv, rk, rG, rU, rW, H, tid, sRk);
}

// LDS of the block-anchor path for one chunk (intra_fwd_block_chunk), carved from a caller's 16-byte aligned
// pool: [R fragments | A] then N, the U/W stage reusing the whole buffer; the k rstd of the rows; the block
// spans; the block anchors.
template <int K, int V>
struct BlockLds {
  static constexpr int KB = K / 32, RBYTES = (C / 16) * KB * TILE * 2, ABYTES = C * AP * 4;
  static constexpr int RABYTES = RBYTES > ABYTES ? RBYTES : ABYTES;
  static constexpr int SBYTES = RABYTES + C * AP * 4 > C * XR * 4 ? RABYTES + C * AP * 4 : C * XR * 4;
  static constexpr int bytes = SBYTES + C * 4 + 16 + 4 * K * 4;
  static_assert(SBYTES % 16 == 0, "16-byte arrays");
};

// The block-anchor path for one chunk intra_fwd_kernel flagged (block 256; lds: BlockLds<K, V>::bytes).
// Returns false, leaving the chunk flagged, when a 16-token block spans more than kBlockSpanMax (the exact
// path takes it); otherwise writes the chunk's outputs and clears its flag.
template <int K, int V, bool ISO, bool NORM>
__device__ __forceinline__ bool intra_fwd_block_chunk(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const float* __restrict__ kap,
    const bf16_t* __restrict__ v, const float* __restrict__ gc, int T, int H, int NT, float scale,
    float* __restrict__ U, float* __restrict__ W, float* __restrict__ Kf, float* __restrict__ Qg,
    float* __restrict__ Mg, float* __restrict__ Ag, int* __restrict__ flags, float* __restrict__ q_rstd,
    float* __restrict__ k_rstd, int n, int bh, unsigned char* lds) {
  constexpr int KB = K / 32;
  using Lds = BlockLds<K, V>;
  constexpr int RABYTES = Lds::RABYTES;
  static_assert(V <= 128 && K <= 128, "operand staging holds up to 128 columns");
  unsigned char* sbuf = lds;
  float* sRk = reinterpret_cast<float*>(lds + Lds::SBYTES);  // in-op L2 norm: the rows' k rstd for the W stage
  bf16_t* sR = reinterpret_cast<bf16_t*>(sbuf);
  float* sA = reinterpret_cast<float*>(sbuf);
  float* sN = reinterpret_cast<float*>(sbuf + RABYTES);
  float* sX = reinterpret_cast<float*>(sbuf);  // U/W stage: operand rows [s][col], pitch XR
  float* sSpan = sRk + C;
  float* sMid = sSpan + 4;  // block anchors m_J per channel
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r16 = lane & 15, g4 = lane >> 4;
  const int b = bh / H, h = bh % H;
  const int64_t lin = (int64_t)bh * NT + n;
  const int t0 = n * C, L = min(C, T - t0);

  // [B,T,H,D] inputs: row c of this chunk at ((b*T + t0 + c)*H + h)*D
  const int64_t in_row0 = ((int64_t)b * T + t0) * H + h;
  const uint32_t rows_in = (uint32_t)((L - 1) * H + 1);  // descriptor covers rows 0..L-1 of this head
  const bufrsrc rG = make_buf(gc + in_row0 * K, rows_in * K * 4);
  const bufrsrc rk = make_buf(k + in_row0 * K, rows_in * K * 2);
  const bufrsrc rq = make_buf(q + in_row0 * K, rows_in * K * 2);
  const bufrsrc rkap = ISO ? make_buf(kap + in_row0, rows_in * 4) : make_buf(kap + in_row0 * K, rows_in * K * 4);
  const bufrsrc rv = make_buf(v + in_row0 * V, rows_in * V * 2);
  // [B*H, T, D] outputs
  const bufrsrc rKf = make_buf(Kf + ((int64_t)bh * T + t0) * K, L * K * 4);
  const bufrsrc rQg = make_buf(Qg + ((int64_t)bh * T + t0) * K, L * K * 4);
  const bufrsrc rU = make_buf(U + ((int64_t)bh * T + t0) * V, L * V * 4);
  const bufrsrc rW = make_buf(W + ((int64_t)bh * T + t0) * K, L * K * 4);
  float* Mn = Mg + ((int64_t)bh * NT + n) * C * C;
  float* An = Ag ? Ag + ((int64_t)bh * NT + n) * C * C : nullptr;

  // ---- 0. block anchors m_J = (G_{16J} + G_{16J+15}) / 2 per channel (rows clamped to the chunk)
  // and the block spans; a chunk with a span past kBlockSpanMax stays for the exact kernel
  {
    float span = 0.f;
#pragma unroll
    for (int e = tid; e < 4 * K; e += 256) {
      const int J = e / K, i = e % K;
      const float ga = buf_ld(rG, ((uint32_t)(min(16 * J, L - 1) * H) * K + i) * 4);
      const float gb = buf_ld(rG, ((uint32_t)(min(16 * J + 15, L - 1) * H) * K + i) * 4);
      sMid[e] = 0.5f * (ga + gb);
      span = fmaxf(span, ga - gb);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) span = fmaxf(span, __shfl_xor(span, o, 64));
    if (lane == 0) sSpan[w] = span;
  }
  __syncthreads();
  const float cspan = fmaxf(fmaxf(sSpan[0], sSpan[1]), fmaxf(sSpan[2], sSpan[3]));
  if (!(cspan <= kBlockSpanMax)) return false;  // left flagged: the exact path takes this chunk

  // ---- 1. per-row factors: wave w owns rows 16w + r16; lanes hold 8 consecutive channels.
  // Rows past L read zero k, q, kappa and repeat the gate of row L-1, so every factor is bounded.
  const int c = 16 * w + r16;
  const uint32_t crow = (uint32_t)(c * H), grow = (uint32_t)(min(c, L - 1) * H);
  uint4 lkh[KB], lkl[KB], lqh[KB], lql[KB];  // k 2^{G - m_I}, scale q 2^{G - m_I} as split fragments
  const float beta = ISO ? buf_ld(rkap, crow * 4) : 0.f;
  float rsq = 1.f, rsk = 1.f;  // in-op L2 norm: this workgroup normalises its rows (as intra_fwd_kernel)
  if constexpr (NORM) {
    u32x4 kraw[KB], qraw[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      kraw[kb] = __builtin_amdgcn_raw_buffer_load_b128(rk, (crow * K + 32 * kb + 8 * g4) * 2, 0, 0);
      qraw[kb] = __builtin_amdgcn_raw_buffer_load_b128(rq, (crow * K + 32 * kb + 8 * g4) * 2, 0, 0);
    }
    rsq = row_rstd<KB>(qraw);
    rsk = row_rstd<KB>(kraw);
    if (g4 == 0) {
      buf_st(make_buf(q_rstd + in_row0, rows_in * 4), crow * 4, rsq);  // rows past L are dropped
      buf_st(make_buf(k_rstd + in_row0, rows_in * 4), crow * 4, rsk);
      sRk[c] = rsk;
    }
  }
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const int i0 = 32 * kb + 8 * g4;
    float gcv[8], gl[8], kv[8], qv[8], av[8];
    ld8(rG, (grow * K + i0) * 4, gcv);
    ld8(rG, ((uint32_t)((L - 1) * H) * K + i0) * 4, gl);
    unpack8(__builtin_amdgcn_raw_buffer_load_b128(rk, (crow * K + i0) * 2, 0, 0), kv);
    unpack8(__builtin_amdgcn_raw_buffer_load_b128(rq, (crow * K + i0) * 2, 0, 0), qv);
    if constexpr (NORM) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        kv[j] = l2n(kv[j], rsk);
        qv[j] = l2n(qv[j], rsq);
      }
    }
    if (ISO) {
#pragma unroll
      for (int j = 0; j < 8; ++j) av[j] = beta * kv[j];
    } else {
      ld8(rkap, (crow * K + i0) * 4, av);
    }
    const float4 m0 = *reinterpret_cast<const float4*>(sMid + w * K + i0);
    const float4 m1 = *reinterpret_cast<const float4*>(sMid + w * K + i0 + 4);
    const float mid[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
    float lk[8], lq[8], rr[8], kf[8], qg[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float e = fexp2(gcv[j] - mid[j]);
      lk[j] = kv[j] * e;
      lq[j] = scale * qv[j] * e;
      rr[j] = av[j] * fexp2(mid[j] - gcv[j]);
      kf[j] = av[j] * fexp2(gl[j] - gcv[j]);
      qg[j] = scale * qv[j] * fexp2(gcv[j]);
    }
    split8(lk, lkh[kb], lkl[kb]);
    split8(lq, lqh[kb], lql[kb]);
    uint4 rh, rl;
    split8(rr, rh, rl);
    *reinterpret_cast<uint4*>(sR + (w * KB + kb) * TILE + lane * 8) = rh;
    *reinterpret_cast<uint4*>(sR + (w * KB + kb) * TILE + 512 + lane * 8) = rl;
    st8(rKf, ((uint32_t)c * K + i0) * 4, kf);
    st8(rQg, ((uint32_t)c * K + i0) * 4, qg);
  }
  __syncthreads();

  // ---- 2. N and M tiles of row block I = w; column block J uses the anchor m_J on both sides
  // (the k side carries 2^{m_I - m_J} <= 1, exactly 1 for J = I)
  const bufrsrc rM = make_buf(Mn, C * C * 4);
  for (int J = w + 1; J < 4; ++J)
#pragma unroll
    for (int j = 0; j < 4; ++j) buf_st(rM, ((16 * w + 4 * g4 + j) * C + 16 * J + r16) * 4, 0.f);
#pragma unroll 1
  for (int J = 0; J <= w; ++J) {
    const int s = 16 * J + r16;
    f32x4 aN = zero4(), aM = zero4();
    if (J == w) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        uint4 rh, rl;
        afrag(sR, J * KB + kb, lane, rh, rl);
        aN = mma3(lkh[kb], lkl[kb], rh, rl, aN);
        aM = mma3(lqh[kb], lql[kb], rh, rl, aM);
      }
    } else {  // the k side times 2^{m_I - m_J} <= 1, re-split
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const int i0 = 32 * kb + 8 * g4;
        const float4 m0 = *reinterpret_cast<const float4*>(sMid + w * K + i0);
        const float4 m1 = *reinterpret_cast<const float4*>(sMid + w * K + i0 + 4);
        const float4 p0 = *reinterpret_cast<const float4*>(sMid + J * K + i0);
        const float4 p1 = *reinterpret_cast<const float4*>(sMid + J * K + i0 + 4);
        const float f[8] = {fexp2(m0.x - p0.x), fexp2(m0.y - p0.y), fexp2(m0.z - p0.z), fexp2(m0.w - p0.w),
                            fexp2(m1.x - p1.x), fexp2(m1.y - p1.y), fexp2(m1.z - p1.z), fexp2(m1.w - p1.w)};
        uint4 xh, xl, rh, rl;
        afrag(sR, J * KB + kb, lane, rh, rl);
        rescale8(lkh[kb], lkl[kb], f, xh, xl);
        aN = mma3(xh, xl, rh, rl, aN);
        rescale8(lqh[kb], lql[kb], f, xh, xl);
        aM = mma3(xh, xl, rh, rl, aM);
        __builtin_amdgcn_sched_barrier(0);  // one k-block at a time
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int cc = 16 * w + 4 * g4 + j;
      sN[cc * AP + s] = (J < w || s < cc) ? aN[j] : 0.f;
      buf_st(rM, (cc * C + s) * 4, (J < w || s <= cc) ? aM[j] : 0.f);
    }
  }
  __syncthreads();

  intra_solve_emit<K, V, NORM>(sA, sN, sX, An, rv, rk, rG, rU, rW, H, tid, sRk);
  if (tid == 0) flags[lin] = 0;
  return true;
}

}  // namespace kdn_intra
