// Serial chunk-state passes of the KDN memory scan (forward and reverse).
//
// One workgroup per (b, h, V-slice of BV columns); the workgroups of one (b, h) are placed
// on one XCD so the chunk operands they all read (W, Kf, Qg, M) are shared through that
// XCD's L2.  The state slice lives in MFMA accumulators; per chunk the next chunk's
// operands are prefetched into registers (16-byte loads) while the current chunk computes.
// Products use bf16x3 split MFMA (v_mfma_f32_16x16x32_bf16 on hi*hi + hi*lo + lo*hi of
// x = hi + lo), which keeps the fp32 state to ~2^-16 relative per product.  LDS operand
// tiles are stored so that every MFMA fragment is one 16-byte read: A tiles [row][k],
// B tiles transposed [col][k].
//
//   forward  (per chunk): h_n = S;  delta = U - W S;  S = e^{g_last} S + Kf^T delta
//   backward (reverse):   dh_n = dS;  d delta = M^T dO + Kf dS;
//                         dS <- e^{g_last} dS + Qg^T dO - W^T d delta
#pragma once
#include "kdn_common.h"

namespace kdn_state {

constexpr int C = 64;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4 mfma_bf16(uint4 a, uint4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}
// a*b with a = ah + al, b = bh + bl, dropping al*bl
__device__ __forceinline__ f32x4 mma3(uint4 ah, uint4 al, uint4 bh, uint4 bl, f32x4 c) {
  c = mfma_bf16(ah, bh, c);
  c = mfma_bf16(ah, bl, c);
  c = mfma_bf16(al, bh, c);
  return c;
}
__device__ __forceinline__ void split(float x, bf16_t& hi, bf16_t& lo) {
  hi = f2bf(x);
  lo = f2bf(x - bf2f(hi));
}
__device__ __forceinline__ uint4 ld16(const bf16_t* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Block -> (bh, V-slice): the NV slices of one (b, h) go to one XCD (dispatch is round-robin
// over the 8 XCDs), when B*H is a multiple of 8.
__device__ __forceinline__ void xcd_map(int lin, int NV, int BH, int& bh, int& vs) {
  if (BH % 8 == 0) {
    const int x = lin & 7, j = lin >> 3;
    bh = x + 8 * (j / NV);
    vs = j % NV;
  } else {
    bh = lin / NV;
    vs = lin % NV;
  }
}

__device__ __forceinline__ int64_t row_bht(int bh, int t, int T, int D) { return ((int64_t)bh * T + t) * D; }
__device__ __forceinline__ int64_t row_bthk(int b, int t, int h, int T, int H, int D) {
  return (((int64_t)b * T + t) * H + h) * D;
}

// Store 4 consecutive values (one float4) split into hi/lo at p_hi[o..o+3], p_lo[o..o+3].
__device__ __forceinline__ void put4_rowmajor(bf16_t* hi, bf16_t* lo, int o, float4 x) {
  bf16_t h0, h1, h2, h3, l0, l1, l2, l3;
  split(x.x, h0, l0);
  split(x.y, h1, l1);
  split(x.z, h2, l2);
  split(x.w, h3, l3);
  *reinterpret_cast<uint2*>(hi + o) = uint2{(uint32_t)h0 | ((uint32_t)h1 << 16), (uint32_t)h2 | ((uint32_t)h3 << 16)};
  *reinterpret_cast<uint2*>(lo + o) = uint2{(uint32_t)l0 | ((uint32_t)l1 << 16), (uint32_t)l2 | ((uint32_t)l3 << 16)};
}
// Store the 4 values of a float4 (consecutive in k) into a transposed tile: p[(k0+q)*ld + r].
__device__ __forceinline__ void put4_transposed(bf16_t* hi, bf16_t* lo, int k0, int ld, int r, float4 x) {
  split(x.x, hi[(k0 + 0) * ld + r], lo[(k0 + 0) * ld + r]);
  split(x.y, hi[(k0 + 1) * ld + r], lo[(k0 + 1) * ld + r]);
  split(x.z, hi[(k0 + 2) * ld + r], lo[(k0 + 2) * ld + r]);
  split(x.w, hi[(k0 + 3) * ld + r], lo[(k0 + 3) * ld + r]);
}

// ===========================================================================
// Forward state pass.  grid (B*H*V/BV), block 256.
// ===========================================================================
template <int K, int V, int BV>
__global__ __launch_bounds__(256) void state_fwd_kernel(const float* __restrict__ U, const float* __restrict__ W,
                                                        const float* __restrict__ Kf, const float* __restrict__ gc,
                                                        const float* __restrict__ h0, int T, int H, int NT, int BH,
                                                        float* __restrict__ hbuf, float* __restrict__ Dl,
                                                        float* __restrict__ ht) {
  constexpr int NV = V / BV;
  constexpr int KH = K + 8, CH = C + 8;
  constexpr int NVB = BV / 16;
  constexpr int STW = (K / 16) * NVB / 4;  // state tiles per wave
  constexpr int DTW = (C / 16) * NVB / 4;  // delta tiles per wave
  constexpr int K4 = K / 4;
  constexpr int PW = C * K4 / 256;  // float4 per thread of one C x K operand
  static_assert((K / 16) * NVB % 4 == 0 && (C / 16) * NVB % 4 == 0, "tile split over 4 waves");
  __shared__ __attribute__((aligned(16))) bf16_t sWh[C * KH], sWl[C * KH];  // W [c][i]
  __shared__ __attribute__((aligned(16))) bf16_t sKh[K * CH], sKl[K * CH];  // Kf^T [i][c]
  __shared__ __attribute__((aligned(16))) bf16_t sSh[BV * KH], sSl[BV * KH];  // S^T [v][i]
  __shared__ __attribute__((aligned(16))) bf16_t sDh[BV * CH], sDl[BV * CH];  // delta^T [v][c]
  __shared__ float sE[K];
  int bh, vs;
  xcd_map(blockIdx.x, NV, BH, bh, vs);
  const int b = bh / H, h = bh % H, v0 = vs * BV;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r16 = lane & 15, q4 = lane >> 4;

  float4 pW[PW], pK[PW];
  float pU[DTW][4];
  float pG = 0.f;
  auto prefetch = [&](int n) {
    const int t0 = n * C, L = min(C, T - t0);
#pragma unroll
    for (int u = 0; u < PW; ++u) {
      const int e4 = tid + 256 * u;
      // W is staged row-major: consecutive lanes walk a row.  Kf is staged transposed:
      // consecutive lanes walk a column, so the transposed LDS stores are contiguous.
      const int cw = e4 / K4, iw = e4 % K4, ck = e4 % C, ik = e4 / C;
      pW[u] = cw < L ? *reinterpret_cast<const float4*>(W + row_bht(bh, t0 + cw, T, K) + 4 * iw)
                     : float4{0.f, 0.f, 0.f, 0.f};
      pK[u] = ck < L ? *reinterpret_cast<const float4*>(Kf + row_bht(bh, t0 + ck, T, K) + 4 * ik)
                     : float4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < DTW; ++u) {
      const int tile = w * DTW + u, cb = tile / NVB, vb = tile % NVB;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int c = 16 * cb + 4 * q4 + j;
        pU[u][j] = c < L ? U[row_bht(bh, t0 + c, T, V) + v0 + 16 * vb + r16] : 0.f;
      }
    }
    if (tid < K) pG = gc[row_bthk(b, t0 + L - 1, h, T, H, K) + tid];
  };

  f32x4 S[STW];
#pragma unroll
  for (int u = 0; u < STW; ++u) {
    const int tile = w * STW + u, ib = tile / NVB, vb = tile % NVB;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = 16 * ib + 4 * q4 + j, vv = 16 * vb + r16;
      const float x = h0 ? h0[((int64_t)bh * K + i) * V + v0 + vv] : 0.f;
      S[u][j] = x;
      split(x, sSh[vv * KH + i], sSl[vv * KH + i]);
    }
  }
  prefetch(0);
  for (int n = 0; n < NT; ++n) {
    const int t0 = n * C, L = min(C, T - t0);
    // stage this chunk's operands
#pragma unroll
    for (int u = 0; u < PW; ++u) {
      const int e4 = tid + 256 * u;
      put4_rowmajor(sWh, sWl, (e4 / K4) * KH + 4 * (e4 % K4), pW[u]);
      put4_transposed(sKh, sKl, 4 * (e4 / C), CH, e4 % C, pK[u]);
    }
    if (tid < K) sE[tid] = exp2f(pG);
    float cU[DTW][4];
#pragma unroll
    for (int u = 0; u < DTW; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) cU[u][j] = pU[u][j];
    __syncthreads();
    if (n + 1 < NT) prefetch(n + 1);
    // h_n = S
#pragma unroll
    for (int u = 0; u < STW; ++u) {
      const int tile = w * STW + u, ib = tile / NVB, vb = tile % NVB;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        hbuf[(((int64_t)bh * NT + n) * K + 16 * ib + 4 * q4 + j) * V + v0 + 16 * vb + r16] = S[u][j];
    }
    // delta = U - W S
    {
      f32x4 acc[DTW];
#pragma unroll
      for (int u = 0; u < DTW; ++u) acc[u] = zero4();
#pragma unroll
      for (int kk = 0; kk < K / 32; ++kk) {
        const int ko = 32 * kk + 8 * q4;
#pragma unroll
        for (int u = 0; u < DTW; ++u) {
          const int tile = w * DTW + u, cb = tile / NVB, vb = tile % NVB;
          const int ra = (16 * cb + r16) * KH + ko, rb = (16 * vb + r16) * KH + ko;
          acc[u] = mma3(ld16(sWh + ra), ld16(sWl + ra), ld16(sSh + rb), ld16(sSl + rb), acc[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < DTW; ++u) {
        const int tile = w * DTW + u, cb = tile / NVB, vb = tile % NVB;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int c = 16 * cb + 4 * q4 + j, vv = 16 * vb + r16;
          const float d = cU[u][j] - acc[u][j];
          if (c < L) Dl[row_bht(bh, t0 + c, T, V) + v0 + vv] = d;
          split(d, sDh[vv * CH + c], sDl[vv * CH + c]);
        }
      }
    }
    __syncthreads();
    // S = e ⊙ S + Kf^T delta
    {
      f32x4 acc[STW];
#pragma unroll
      for (int u = 0; u < STW; ++u) {
        const int tile = w * STW + u, ib = tile / NVB;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[u][j] = sE[16 * ib + 4 * q4 + j] * S[u][j];
      }
#pragma unroll
      for (int kk = 0; kk < C / 32; ++kk) {
        const int ko = 32 * kk + 8 * q4;
#pragma unroll
        for (int u = 0; u < STW; ++u) {
          const int tile = w * STW + u, ib = tile / NVB, vb = tile % NVB;
          const int ra = (16 * ib + r16) * CH + ko, rb = (16 * vb + r16) * CH + ko;
          acc[u] = mma3(ld16(sKh + ra), ld16(sKl + ra), ld16(sDh + rb), ld16(sDl + rb), acc[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < STW; ++u) S[u] = acc[u];
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < STW; ++u) {
      const int tile = w * STW + u, ib = tile / NVB, vb = tile % NVB;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = 16 * ib + 4 * q4 + j, vv = 16 * vb + r16;
        split(S[u][j], sSh[vv * KH + i], sSl[vv * KH + i]);
      }
    }
  }
  if (ht) {
#pragma unroll
    for (int u = 0; u < STW; ++u) {
      const int tile = w * STW + u, ib = tile / NVB, vb = tile % NVB;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        ht[((int64_t)bh * K + 16 * ib + 4 * q4 + j) * V + v0 + 16 * vb + r16] = S[u][j];
    }
  }
}

// ===========================================================================
// Reverse state pass.  grid (B*H*V/BV), block 256.
// ===========================================================================
template <int K, int V, int BV, typename TDO>
__global__ __launch_bounds__(256) void state_bwd_kernel(const float* __restrict__ Mg, const float* __restrict__ Kf,
                                                        const float* __restrict__ Qg, const float* __restrict__ W,
                                                        const float* __restrict__ gc, const TDO* __restrict__ dO,
                                                        const float* __restrict__ dht, int T, int H, int NT, int BH,
                                                        float* __restrict__ dhbuf, float* __restrict__ dDl,
                                                        float* __restrict__ dh0) {
  constexpr int NV = V / BV;
  constexpr int KH = K + 8, CH = C + 8;
  constexpr int NVB = BV / 16;
  constexpr int STW = (K / 16) * NVB / 4;
  constexpr int DTW = (C / 16) * NVB / 4;
  constexpr int K4 = K / 4;
  constexpr int PW = C * K4 / 256;
  constexpr int PM = C * C / 4 / 256;         // float4 per thread of M
  constexpr int PO = C * BV / 256;            // dO values per thread
  static_assert(PO >= 1 && C * BV % 256 == 0, "dO staging");
  __shared__ __attribute__((aligned(16))) bf16_t sKh[C * KH], sKl[C * KH];   // Kf [c][i]
  __shared__ __attribute__((aligned(16))) bf16_t sQh[K * CH], sQl[K * CH];   // Qg^T [i][c]
  __shared__ __attribute__((aligned(16))) bf16_t sWh[K * CH], sWl[K * CH];   // W^T [i][c]
  __shared__ __attribute__((aligned(16))) bf16_t sMh[C * CH], sMl[C * CH];   // M^T [c][c']
  __shared__ __attribute__((aligned(16))) bf16_t sOh[BV * CH], sOl[BV * CH]; // dO^T [v][c]
  __shared__ __attribute__((aligned(16))) bf16_t sSh[BV * KH], sSl[BV * KH]; // dS^T [v][i]
  __shared__ __attribute__((aligned(16))) bf16_t sDh[BV * CH], sDl[BV * CH]; // d delta^T [v][c]
  __shared__ float sE[K];
  int bh, vs;
  xcd_map(blockIdx.x, NV, BH, bh, vs);
  const int b = bh / H, h = bh % H, v0 = vs * BV;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r16 = lane & 15, q4 = lane >> 4;

  float4 pK[PW], pQ[PW], pW[PW], pM[PM];
  float pO[PO];
  float pG = 0.f;
  auto prefetch = [&](int n) {
    const int t0 = n * C, L = min(C, T - t0);
#pragma unroll
    for (int u = 0; u < PW; ++u) {
      const int e4 = tid + 256 * u;
      // Kf is staged row-major (lanes walk a row); Qg and W transposed (lanes walk a column).
      const int cr = e4 / K4, ir = e4 % K4, cc = e4 % C, ic = e4 / C;
      const float4 z = float4{0.f, 0.f, 0.f, 0.f};
      pK[u] = cr < L ? *reinterpret_cast<const float4*>(Kf + row_bht(bh, t0 + cr, T, K) + 4 * ir) : z;
      const int64_t oc = row_bht(bh, t0 + cc, T, K) + 4 * ic;
      pQ[u] = cc < L ? *reinterpret_cast<const float4*>(Qg + oc) : z;
      pW[u] = cc < L ? *reinterpret_cast<const float4*>(W + oc) : z;
    }
    const float* Mn = Mg + ((int64_t)bh * NT + n) * C * C;
#pragma unroll
    for (int u = 0; u < PM; ++u) {  // M[cp][4 c4 .. 4 c4 + 3], lanes walk cp
      const int e4 = tid + 256 * u, cp = e4 % C, c4 = e4 / C;
      pM[u] = *reinterpret_cast<const float4*>(Mn + cp * C + 4 * c4);
    }
#pragma unroll
    for (int u = 0; u < PO; ++u) {
      const int e = tid + 256 * u, c = e / BV, vv = e % BV;
      pO[u] = c < L ? ld(dO, row_bthk(b, t0 + c, h, T, H, V) + v0 + vv) : 0.f;
    }
    if (tid < K) pG = gc[row_bthk(b, t0 + L - 1, h, T, H, K) + tid];
  };

  f32x4 dS[STW];
#pragma unroll
  for (int u = 0; u < STW; ++u) {
    const int tile = w * STW + u, ib = tile / NVB, vb = tile % NVB;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = 16 * ib + 4 * q4 + j, vv = 16 * vb + r16;
      const float x = dht ? dht[((int64_t)bh * K + i) * V + v0 + vv] : 0.f;
      dS[u][j] = x;
      split(x, sSh[vv * KH + i], sSl[vv * KH + i]);
    }
  }
  prefetch(NT - 1);
  for (int n = NT - 1; n >= 0; --n) {
    const int t0 = n * C, L = min(C, T - t0);
#pragma unroll
    for (int u = 0; u < PW; ++u) {
      const int e4 = tid + 256 * u;
      put4_rowmajor(sKh, sKl, (e4 / K4) * KH + 4 * (e4 % K4), pK[u]);
      put4_transposed(sQh, sQl, 4 * (e4 / C), CH, e4 % C, pQ[u]);
      put4_transposed(sWh, sWl, 4 * (e4 / C), CH, e4 % C, pW[u]);
    }
#pragma unroll
    for (int u = 0; u < PM; ++u) {
      const int e4 = tid + 256 * u;
      put4_transposed(sMh, sMl, 4 * (e4 / C), CH, e4 % C, pM[u]);  // M^T [c][cp]
    }
#pragma unroll
    for (int u = 0; u < PO; ++u) {
      const int e = tid + 256 * u, c = e / BV, vv = e % BV;
      split(pO[u], sOh[vv * CH + c], sOl[vv * CH + c]);
    }
    if (tid < K) sE[tid] = exp2f(pG);
    __syncthreads();
    if (n > 0) prefetch(n - 1);
#pragma unroll
    for (int u = 0; u < STW; ++u) {
      const int tile = w * STW + u, ib = tile / NVB, vb = tile % NVB;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        dhbuf[(((int64_t)bh * NT + n) * K + 16 * ib + 4 * q4 + j) * V + v0 + 16 * vb + r16] = dS[u][j];
    }
    // d delta = M^T dO + Kf dS
    {
      f32x4 acc[DTW];
#pragma unroll
      for (int u = 0; u < DTW; ++u) acc[u] = zero4();
#pragma unroll
      for (int kk = 0; kk < C / 32; ++kk) {
        const int ko = 32 * kk + 8 * q4;
#pragma unroll
        for (int u = 0; u < DTW; ++u) {
          const int tile = w * DTW + u, cb = tile / NVB, vb = tile % NVB;
          if (32 * kk + 32 > 16 * cb) {  // M^T[c][c'] = 0 for c' < c
            const int ra = (16 * cb + r16) * CH + ko, rb = (16 * vb + r16) * CH + ko;
            acc[u] = mma3(ld16(sMh + ra), ld16(sMl + ra), ld16(sOh + rb), ld16(sOl + rb), acc[u]);
          }
        }
      }
#pragma unroll
      for (int kk = 0; kk < K / 32; ++kk) {
        const int ko = 32 * kk + 8 * q4;
#pragma unroll
        for (int u = 0; u < DTW; ++u) {
          const int tile = w * DTW + u, cb = tile / NVB, vb = tile % NVB;
          const int ra = (16 * cb + r16) * KH + ko, rb = (16 * vb + r16) * KH + ko;
          acc[u] = mma3(ld16(sKh + ra), ld16(sKl + ra), ld16(sSh + rb), ld16(sSl + rb), acc[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < DTW; ++u) {
        const int tile = w * DTW + u, cb = tile / NVB, vb = tile % NVB;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int c = 16 * cb + 4 * q4 + j, vv = 16 * vb + r16;
          const float d = acc[u][j];
          if (c < L) dDl[row_bht(bh, t0 + c, T, V) + v0 + vv] = d;
          split(d, sDh[vv * CH + c], sDl[vv * CH + c]);
        }
      }
    }
    __syncthreads();
    // dS <- e dS + Qg^T dO - W^T d delta
    {
      f32x4 accP[STW], accW[STW];
#pragma unroll
      for (int u = 0; u < STW; ++u) {
        const int tile = w * STW + u, ib = tile / NVB;
#pragma unroll
        for (int j = 0; j < 4; ++j) accP[u][j] = sE[16 * ib + 4 * q4 + j] * dS[u][j];
        accW[u] = zero4();
      }
#pragma unroll
      for (int kk = 0; kk < C / 32; ++kk) {
        const int ko = 32 * kk + 8 * q4;
#pragma unroll
        for (int u = 0; u < STW; ++u) {
          const int tile = w * STW + u, ib = tile / NVB, vb = tile % NVB;
          const int ra = (16 * ib + r16) * CH + ko, rb = (16 * vb + r16) * CH + ko;
          accP[u] = mma3(ld16(sQh + ra), ld16(sQl + ra), ld16(sOh + rb), ld16(sOl + rb), accP[u]);
          accW[u] = mma3(ld16(sWh + ra), ld16(sWl + ra), ld16(sDh + rb), ld16(sDl + rb), accW[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < STW; ++u)
#pragma unroll
        for (int j = 0; j < 4; ++j) dS[u][j] = accP[u][j] - accW[u][j];
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < STW; ++u) {
      const int tile = w * STW + u, ib = tile / NVB, vb = tile % NVB;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = 16 * ib + 4 * q4 + j, vv = 16 * vb + r16;
        split(dS[u][j], sSh[vv * KH + i], sSl[vv * KH + i]);
      }
    }
  }
  if (dh0) {
#pragma unroll
    for (int u = 0; u < STW; ++u) {
      const int tile = w * STW + u, ib = tile / NVB, vb = tile % NVB;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        dh0[((int64_t)bh * K + 16 * ib + 4 * q4 + j) * V + v0 + 16 * vb + r16] = dS[u][j];
    }
  }
}

}  // namespace kdn_state
