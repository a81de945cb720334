// Chunk-parallel backward of the KDN memory scan on bf16x3 MFMA (one kernel per chunk).
//
// Per chunk of C = 64 tokens (h = state entering the chunk, dh = gradient of the state leaving
// it, delta / d delta = the chunk's delta and its gradient, A = (I + N)^{-1} saved by the forward):
//   state-gradient products  dQg = dO h^T,  dW = -d delta h^T,  dKf = delta dh^T,
//                            dM = lower(dO delta^T),  dgl_i = 2^{G_last,i} sum_v h_iv dh_iv
//   transposed solves        dV = A^T d delta,  dKg = A^T dW,  dN = -strict_lower(dV U^T + dKg W^T)
//   gradients                with block anchors m (below): e = 2^{G_c - m}, Lk = k e, Lq = q e,
//                            R = kappa / e, eg = 2^{G_c}, f = 2^{G_last - G_c}
//                            dLk = dN R,  dLq = scale dM R,  dR = dN^T Lk + scale dM^T Lq
//                            dk = dLk e + dKg eg,  dq = dLq e + scale dQg eg,  dkappa = dR / e + dKf f
//                            dg = Lk dLk + Lq dLq - R dR + k eg dKg + scale q eg dQg - kappa f dKf
//                            dg[last row] += sum_c kappa f dKf + dgl;  iso: dbeta = sum_i dkappa k,
//                            dk += beta dkappa
// dg is in natural-log coordinates.  Each output row block tl uses the forward's anchor of that block,
// m = (G_{16tl} + G_{16tl+15}) / 2 per channel (rows clamped to the chunk), for every factor it
// contracts with, so each factor is <= 2^{span/2} on the diagonal block and <= 1 off it; the anchor
// terms cancel exactly (N and M do not depend on the anchors) and are omitted.
#pragma once
#include "kdn_common.h"
#include "kdn_intra.h"
#include "kdn_state.h"

namespace kdn_bwd {

using kdn_intra::ld8;
using kdn_intra::split8;
using kdn_intra::unpack8;
using kdn_state::C;
using kdn_state::mfma;
using kdn_state::mma3;
using kdn_state::zero4;
using kdn_state::afrag;
using kdn_state::TILE;

// a*b with a exact in bf16 (A operand) and b = bh + bl split (B operand)
__device__ __forceinline__ f32x4 mma2b(uint4 a, uint4 bh, uint4 bl, f32x4 c) {
  c = mfma(a, bh, c);
  c = mfma(a, bl, c);
  return c;
}
// a*b where each operand is split (hi + lo, AL / BL) or exact in bf16 (hi only): hi*hi, hi*lo, lo*hi
// in the order of mma3, dropping the terms of an absent lo half.
template <bool AL, bool BL>
__device__ __forceinline__ f32x4 mmx(uint4 ah, uint4 al, uint4 bh, uint4 bl, f32x4 c) {
  c = mfma(ah, bh, c);
  if constexpr (BL) c = mfma(ah, bl, c);
  if constexpr (AL) c = mfma(al, bh, c);
  return c;
}
// a staged fragment; without LO the tensor was staged as its bf16 values alone (lo = 0)
template <bool LO>
__device__ __forceinline__ void afragx(const bf16_t* buf, int tile, int lane, uint4& hi, uint4& lo) {
  hi = *reinterpret_cast<const uint4*>(buf + tile * TILE + lane * 8);
  if constexpr (LO) lo = *reinterpret_cast<const uint4*>(buf + tile * TILE + 512 + lane * 8);
  else lo = uint4{0u, 0u, 0u, 0u};
}

// Lower 16x16 tiles (I, J), J <= I, 2-bit packed: 0:(0,0) 1:(1,1) 2:(2,2) 3:(3,3) 4:(1,0)
// 5:(2,1) 6:(3,2) 7:(2,0) 8:(3,1) 9:(3,0); upper tiles (0,1) (0,2) (0,3) (1,2) (1,3) (2,3).
__device__ __forceinline__ void lower_tile(int t, int& I, int& J) {
  I = (0xfb9e4u >> (2 * t)) & 3;
  J = (0x124e4u >> (2 * t)) & 3;
}
__device__ __forceinline__ void upper_tile(int t, int& I, int& J) {
  I = (0x940u >> (2 * t)) & 3;
  J = (0xfb9u >> (2 * t)) & 3;
}

// index of lower tile (I, J) in the order of lower_tile
__device__ __forceinline__ int lower_tile_index(int I, int J) {
  const int d = I - J;
  return d == 0 ? I : d == 1 ? 4 + J : d == 2 ? 7 + J : 9;
}

// ---------------------------------------------------------------------------------------------
// The whole chunk-parallel backward of one chunk in one kernel: the state-gradient products, the
// transposed solves and the gradients.  dQg, dW, dKf, dM, dKg, dN and the g_last dots never go to
// HBM: each is produced in the register or LDS layout its consumer takes.
// One chunk-head task of the order task = (NT - 1 - n) * B*H + bh (last chunks first, the order in
// which the reverse state pass finishes them); block 512 (8 waves), one workgroup per CU (LDS ~106 KB).
//  * Staging.  The chunk rows of dO, delta and d delta are split into LDS fragments (rows c,
//    k = v, natural order), all 64 rows at once.
//  * Wave w owns channel tile it = w (16 channels of K) and V tile w (16 columns of V).  It loads
//    its 16 rows of h and of dh straight into split fragments (one layout serves as the A operand
//    h (rows i, k = v) and as the B operand h^T (k = v, cols i)) and forms
//      dQg^T = h dO^T,  dKf^T = dh delta^T    (D tile: lane -> chunk row, 4 consecutive channels:
//                                              the layout of the gradient phase's elementwise terms)
//      -dW   = d delta h^T                    (D tile: lane -> channel, 4 chunk rows: two stacked
//                                              tiles are the solve's A operand in permuted k order)
//      dgl_i = 2^{G_last,i} sum_v h_iv dh_iv,  and dM = lower(dO delta^T) for lower tiles w, w + 8.
//  * Solve.  Per wave one 32-column block: its V tile of d delta (dv stored) and its K tile of dW
//    (dKg kept in registers), with A^T read in the same permuted k order; the block's dN^T share
//    over the 8 waves is summed through LDS in two steps (waves 4..7 into 0..3, then the four).
//  * Gradients.  dN, dM and their transposes are split once into LDS fragments (permuted k order:
//    slot 4h + j of lane group g <-> k = 32 kb + 16 h + 4 g + j).  Per channel tile the factors R,
//    Lk, Lq are built per lane for one channel and 16 chunk rows (rows outside the contraction's
//    nonzero range zeroed) and enter the time contractions as the A operand, with the dN / dM
//    fragments as B: the D tiles give each lane 4 consecutive channels of one chunk row, the layout
//    of dQg, dKf and dKg, so the elementwise inputs and outputs move as 16-byte (fp32) and 8-byte
//    (bf16) vectors.
// Chunks flagged by the forward store the products (dQg, dW, dKf, dM, dgl) for the exact kernels
// and stop after them.
// ---------------------------------------------------------------------------------------------
template <int K, int V, bool ISO, typename TDO, int HM>
__device__ __forceinline__ void chunk_bwd_task(
    int task, const void* __restrict__ hbuf, const void* __restrict__ dhbuf, const void* __restrict__ Dl,
    const void* __restrict__ dDl, const TDO* __restrict__ dO, const float* __restrict__ At,
    const float* __restrict__ U, const float* __restrict__ W, const int* __restrict__ flags,
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const float* __restrict__ kap,
    const float* __restrict__ gc, const float* __restrict__ q_rstd, const float* __restrict__ k_rstd, int T, int H,
    int NT, int BH, float scale, bf16_t* __restrict__ dv, bf16_t* __restrict__ dq, bf16_t* __restrict__ dk,
    float* __restrict__ dkap, float* __restrict__ dbeta, float* __restrict__ dg, float* __restrict__ xQg,
    float* __restrict__ xW, float* __restrict__ xKf, float* __restrict__ xM, float* __restrict__ xgl) {
  constexpr bool DO_BF16 = sizeof(TDO) == 2;
  // HM: which of h, dh, delta, d delta were stored in bf16 (kdn_state::HB_*; the recurrences ran in
  // fp32 and rounded those copies once).  A bf16 operand enters a product without a lo half: one
  // MFMA against another bf16 operand, two against a split fp32 one.
  constexpr bool LH = !(HM & kdn_state::HB_H), LDH = !(HM & kdn_state::HB_DH);  // fp32 (split) copies
  constexpr bool LD = !(HM & kdn_state::HB_D), LDD = !(HM & kdn_state::HB_DD);
  constexpr bool LO_ = !DO_BF16;
  constexpr int EH = LH ? 4 : 2, EDH = LDH ? 4 : 2, ED = LD ? 4 : 2, EDD = LDD ? 4 : 2;  // bytes per element
  constexpr int NW = 8;
  constexpr int VB = V / 32;        // k-blocks of the V contraction
  constexpr int NIT = K / 16;       // channel tiles (waves 0 .. NIT-1 own one each)
  constexpr int NVT = V / 16;       // V tiles (waves 0 .. NVT-1)
  constexpr int RB = VB * TILE;     // one 16-row block of a [rows][V] operand as fragments
  constexpr int FR = 8 * TILE;      // one 64 x 64 operand as (4 row tiles x 2 k-blocks) fragments
  constexpr int AP4 = C + 4;        // LDS row stride of A^T (and of dM while it is passed on)
  constexpr int STAGE_BYTES = 3 * 4 * RB * 2;
  constexpr int SOLVE_BYTES = (C * AP4 + 2 * 4 * 10 * 256) * 4;
  constexpr int CONTRIB_BYTES = 4 * FR * 2;
  constexpr int LDS_A = STAGE_BYTES > SOLVE_BYTES ? STAGE_BYTES : SOLVE_BYTES;
  constexpr int LDS_BYTES = LDS_A > CONTRIB_BYTES ? LDS_A : CONTRIB_BYTES;
  constexpr int SU = C * V / 8 / 512;  // staging units (8 consecutive v of one row) per thread per operand
  static_assert(SU >= 1 && (C * V / 8) % 512 == 0, "staging units per thread");
  static_assert(NIT <= NW && NVT <= NW, "K, V <= 128");
  __shared__ __attribute__((aligned(16))) unsigned char smem[LDS_BYTES];
  __shared__ float sDgl[K];
  __shared__ float sBeta[NW * C];
  __shared__ float sDot[2][NW][C];  // in-op L2 norm: per-wave partial row dots y . dy of q and k
  __shared__ float sRs[2][C];       // ... and the rows' rstd of q and k (their raw values in memory)
  __shared__ float sBt[ISO ? C : 1];  // iso: the rows' beta (0 past L), for the gradient phase
  bf16_t* sO = reinterpret_cast<bf16_t*>(smem);  // phase 1: dO, delta, d delta row fragments
  bf16_t* sD = sO + 4 * RB;
  bf16_t* sdD = sD + 4 * RB;
  float* sAt = reinterpret_cast<float*>(smem);   // solve: A^T [C][AP4]
  float* sP = sAt + C * AP4;                      // per-wave partial dN^T tiles (4 slots)
  float* sP2 = sP + 4 * 10 * 256;                 // ... and the same partials transposed (dN tiles)
  bf16_t* sF = reinterpret_cast<bf16_t*>(smem);  // gradients: dN, dM, dN^T, dM^T fragments
  const int n = NT - 1 - task / BH, bh = task % BH, b = bh / H, h = bh % H;
  const int t0 = n * C, L = min(C, T - t0);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r16 = lane & 15, g4 = lane >> 4;
  const int64_t chunk = (int64_t)bh * NT + n;
  const bool flagged = flags[chunk] != 0;
  const bool own_k = w < NIT, own_v = w < NVT;
  const int it = w;  // this wave's channel tile (when own_k)
  const int i0 = 16 * it + 4 * g4;
  if (q_rstd && tid < 2 * C) {  // read in the gradient phase, after phase 1's barriers
    const int c = tid & 63;
    sRs[tid >> 6][c] = c < L ? ((tid >> 6) ? k_rstd : q_rstd)[((int64_t)b * T + t0 + c) * H + h] : 0.f;
  }
  if (ISO && tid >= 2 * C && tid < 3 * C) {  // read in the gradient phase, after phase 1's barriers
    const int c = tid - 2 * C;
    sBt[ISO ? c : 0] = c < L ? kap[((int64_t)b * T + t0 + c) * H + h] : 0.f;
  }

  // ================================ loads ================================
  const int64_t row0 = ((int64_t)bh * T + t0) * V;
  const bufrsrc rD = make_buf(reinterpret_cast<const char*>(Dl) + row0 * ED, L * V * ED);  // rows past L read 0
  const bufrsrc rdD = make_buf(reinterpret_cast<const char*>(dDl) + row0 * EDD, L * V * EDD);
  const bufrsrc rO = make_buf(dO + (((int64_t)b * T + t0) * H + h) * V, ((L - 1) * H + 1) * V * sizeof(TDO));
  float4 sr_D[SU][2], sr_dD[SU][2];
  u32x4 sr_D16[SU], sr_dD16[SU];
  u32x4 sr_O[SU][DO_BF16 ? 1 : 2];
#pragma unroll
  for (int u = 0; u < SU; ++u) {  // unit e: 16-row block, k-block, fragment lane
    const int e = tid + 512 * u, blk = e / (VB * 64), kb = (e / 64) % VB, sl = e & 63;
    const uint32_t c = (uint32_t)(16 * blk + (sl & 15)), v0 = (uint32_t)(32 * kb + 8 * (sl >> 4));
    if constexpr (LD) {
      sr_D[u][0] = buf_ld4(rD, (c * V + v0) * 4);
      sr_D[u][1] = buf_ld4(rD, (c * V + v0) * 4 + 16);
    } else {
      sr_D16[u] = __builtin_amdgcn_raw_buffer_load_b128(rD, (c * V + v0) * 2, 0, 0);
    }
    if constexpr (LDD) {
      sr_dD[u][0] = buf_ld4(rdD, (c * V + v0) * 4);
      sr_dD[u][1] = buf_ld4(rdD, (c * V + v0) * 4 + 16);
    } else {
      sr_dD16[u] = __builtin_amdgcn_raw_buffer_load_b128(rdD, (c * V + v0) * 2, 0, 0);
    }
    if constexpr (DO_BF16) {
      sr_O[u][0] = __builtin_amdgcn_raw_buffer_load_b128(rO, (c * H * V + v0) * 2, 0, 0);
    } else {
      sr_O[u][0] = __builtin_amdgcn_raw_buffer_load_b128(rO, (c * H * V + v0) * 4, 0, 0);
      sr_O[u][1] = __builtin_amdgcn_raw_buffer_load_b128(rO, (c * H * V + v0) * 4 + 16, 0, 0);
    }
  }
  // this wave's rows of h and dh (row i = 16 it + r16, v = 32 kb + 8 g4 .. + 7) and the g_last factor
  const bufrsrc rh = make_buf(reinterpret_cast<const char*>(hbuf) + chunk * K * V * EH, K * V * EH);
  const bufrsrc rdh = make_buf(reinterpret_cast<const char*>(dhbuf) + chunk * K * V * EDH, K * V * EDH);
  float hv[VB][8], dhv[VB][8];
  u32x4 hr[VB], dhr[VB];  // bf16 copies: the rows are the MFMA fragments themselves
  float gl_i = 0.f;
  if (own_k) {
    const int i = 16 * it + r16;
#pragma unroll
    for (int kb = 0; kb < VB; ++kb) {
      // the state passes' tiled layout (kdn_state::hb_off): 8 consecutive columns are contiguous
      const uint32_t et = kdn_state::hb_off<K>(i, 32 * kb + 8 * g4);
      if constexpr (LH) kdn_intra::ld8(rh, et * 4, hv[kb]);
      else hr[kb] = __builtin_amdgcn_raw_buffer_load_b128(rh, et * 2, 0, 0);
      if constexpr (LDH) kdn_intra::ld8(rdh, et * 4, dhv[kb]);
      else dhr[kb] = __builtin_amdgcn_raw_buffer_load_b128(rdh, et * 2, 0, 0);
    }
    gl_i = buf_ld(make_buf(gc + (((int64_t)b * T + t0 + L - 1) * H + h) * K, K * 4), i * 4);
  }
  // A^T of the chunk (staged for the solve once the phase-1 fragments are dead)
  constexpr int AU = C * C / 4 / 512;
  float4 at_r[AU];
  if (!flagged) {
    const bufrsrc rA = make_buf(At + chunk * C * C, C * C * 4);
#pragma unroll
    for (int u = 0; u < AU; ++u) at_r[u] = buf_ld4(rA, (tid + 512 * u) * 16);
  }
  // Diagonal variant, K = 128: the chunk's k and q rows for the gradient phase go straight from memory
  // into LDS (buffer loads with the LDS flag: no registers held), issued with the solve's U / W rows,
  // so they arrive during phase 1 and the solve instead of as per-channel gathers in the gradient
  // phase (diag step -30 us; the isotropic variant, whose gradient phase loads less, measured 7 us
  // slower with it and keeps the gathers).
  // One instruction moves 64 lanes x 16 B = 4 rows of 256 B; row c of tensor x sits at
  // x * QK_T + (c / 4) * QK_S + (c % 4) * 256 bytes.  The 64-byte gap after each 4-row group puts the
  // rows 4 apart, which one gradient-phase read gathers, on different banks.  Rows past L read 0.
  constexpr bool QK_LDS = K == 128 && !ISO;
  constexpr int QK_S = 4 * K * 2 + 64, QK_T = (C / 4) * QK_S;
  __shared__ __attribute__((aligned(16))) unsigned char sQK[QK_LDS ? 2 * QK_T : 16];
  const int64_t in_row0 = ((int64_t)b * T + t0) * H + h;
  const uint32_t rows_in = (uint32_t)((L - 1) * H + 1);
  auto issue_qk = [&]() {
    if constexpr (QK_LDS) {
      if (!flagged) {
        const bufrsrc rkq[2] = {make_buf(k + in_row0 * K, rows_in * K * 2),
                                make_buf(q + in_row0 * K, rows_in * K * 2)};
        const int wu = __builtin_amdgcn_readfirstlane(w);
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int gi = 0; gi < C / 4 / NW; ++gi) {  // wave w: 4-row groups NW gi + w
            const int grp = NW * gi + wu, c = 4 * grp + (lane >> 4);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rkq[x], (__attribute__((address_space(3))) void*)(sQK + x * QK_T + grp * QK_S), 16,
                (uint32_t)((c * H * K + 8 * (lane & 15)) * 2), 0, 0, 0);
          }
      }
    }
  };
  auto qk_lds = [&](int x, int c, int ch) -> const unsigned char* {
    return sQK + x * QK_T + (c >> 2) * QK_S + (c & 3) * (K * 2) + ch * 2;
  };
  // Isotropic variant, K = 128: the chunk's gate rows G (fp32) for the gradient phase go to LDS the same way,
  // issued with the k, q rows' slot: one instruction moves 64 lanes x 16 B = 2 rows of 512 B, and row c sits at
  // (c / 2) * G_S + (c % 2) * 512 bytes.  The 32-byte gap after each pair puts the rows 4 apart, which one
  // gradient-phase read gathers, on different banks.  Rows past L read 0; the reads clamp to row L - 1.
  constexpr bool G_LDS = K == 128 && ISO;
  constexpr int G_S = 2 * K * 4 + 32, G_T = (C / 2) * G_S;
  __shared__ __attribute__((aligned(16))) unsigned char sGr[G_LDS ? G_T : 16];
  auto issue_g = [&]() {
    if constexpr (G_LDS) {
      if (!flagged) {
        const bufrsrc rg = make_buf(gc + in_row0 * K, rows_in * K * 4);
        const int wu = __builtin_amdgcn_readfirstlane(w);
#pragma unroll
        for (int gi = 0; gi < C / 2 / NW; ++gi) {  // wave w: row pairs NW gi + w
          const int pr = NW * gi + wu, c = 2 * pr + (lane >> 5);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rg, (__attribute__((address_space(3))) void*)(sGr + pr * G_S), 16,
                                                   (uint32_t)((c * H * K + 4 * (lane & 31)) * 4), 0, 0, 0);
        }
      }
    }
  };
  auto g_lds = [&](int c, int ch) -> const float* {
    return reinterpret_cast<const float*>(sGr + (c >> 1) * G_S + (c & 1) * (K * 4) + ch * 4);
  };

  // ---- phase-1 fragments into LDS
#pragma unroll
  for (int u = 0; u < SU; ++u) {
    const int e = tid + 512 * u, blk = e / (VB * 64), kb = (e / 64) % VB, sl = e & 63;
    const int off = blk * RB + kb * TILE + sl * 8;
    auto put8 = [&](bf16_t* dst, const float4& x0, const float4& x1) {
      const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      uint4 hi, lo;
      split8(x, hi, lo);
      *reinterpret_cast<uint4*>(dst + off) = hi;
      *reinterpret_cast<uint4*>(dst + off + 512) = lo;
    };
    // a bf16 copy is staged as its values alone (the lo half stays unused)
    if constexpr (LD) put8(sD, sr_D[u][0], sr_D[u][1]);
    else *reinterpret_cast<uint4*>(sD + off) = __builtin_bit_cast(uint4, sr_D16[u]);
    if constexpr (LDD) put8(sdD, sr_dD[u][0], sr_dD[u][1]);
    else *reinterpret_cast<uint4*>(sdD + off) = __builtin_bit_cast(uint4, sr_dD16[u]);
    if constexpr (DO_BF16)
      *reinterpret_cast<uint4*>(sO + off) = uint4{sr_O[u][0].x, sr_O[u][0].y, sr_O[u][0].z, sr_O[u][0].w};
    else
      put8(sO, __builtin_bit_cast(float4, sr_O[u][0]), __builtin_bit_cast(float4, sr_O[u][1]));
  }
  __syncthreads();

  // ================================ phase 1: products with h, dh ================================
  // the solve's rows of U (V tile w) and W (K tile w), issued once phase 1's operands have arrived so
  // they load during its products (issued with those operands they delay them; after the solve's
  // products their latency is exposed).  Zero-size descriptors read 0 for a wave without the tile.
  float4 uw[4][2];
  {
    const bufrsrc rUv = make_buf(U + ((int64_t)bh * T + t0) * V, own_v ? L * V * 4 : 0u);
    const bufrsrc rWk = make_buf(W + ((int64_t)bh * T + t0) * K, own_k ? L * K * 4 : 0u);
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      const uint32_t sr = (uint32_t)(16 * J + r16);
      uw[J][0] = buf_ld4(rUv, (sr * V + 16 * w + 4 * g4) * 4);
      uw[J][1] = buf_ld4(rWk, (sr * K + i0) * 4);
    }
  }
  issue_qk();  // after phase 1's operands, like the U / W rows
  issue_g();
  f32x4 aQ[4], aW[4], aK[4];  // dQg^T (rows i, cols c), d delta h^T (rows c, cols i), dKf^T
#pragma unroll
  for (int tl = 0; tl < 4; ++tl) aQ[tl] = aW[tl] = aK[tl] = zero4();
  if (own_k) {
    uint4 fh[VB], fl[VB];  // h (split, or its bf16 values)
#pragma unroll
    for (int kb = 0; kb < VB; ++kb) {
      if constexpr (LH) split8(hv[kb], fh[kb], fl[kb]);
      else fh[kb] = __builtin_bit_cast(uint4, hr[kb]), fl[kb] = uint4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int kb = 0; kb < VB; ++kb)
#pragma unroll
      for (int tl = 0; tl < 4; ++tl) {
        uint4 oh, ol, xh, xl;
        afragx<LO_>(sO + tl * RB, kb, lane, oh, ol);
        aQ[tl] = mmx<LH, LO_>(fh[kb], fl[kb], oh, ol, aQ[tl]);
        afragx<LDD>(sdD + tl * RB, kb, lane, xh, xl);
        aW[tl] = mmx<LDD, LH>(xh, xl, fh[kb], fl[kb], aW[tl]);
      }
    float dot = 0.f;
#pragma unroll
    for (int kb = 0; kb < VB; ++kb) {
      float hf[8], df[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) hf[j] = hv[kb][j], df[j] = dhv[kb][j];
      if constexpr (!LH) kdn_intra::unpack8(hr[kb], hf);
      if constexpr (!LDH) kdn_intra::unpack8(dhr[kb], df);
#pragma unroll
      for (int j = 0; j < 8; ++j) dot += hf[j] * df[j];
      if constexpr (LDH) split8(dhv[kb], fh[kb], fl[kb]);  // fh, fl: dh from here on
      else fh[kb] = __builtin_bit_cast(uint4, dhr[kb]), fl[kb] = uint4{0u, 0u, 0u, 0u};
    }
    dot += __shfl_xor(dot, 16, 64);
    dot += __shfl_xor(dot, 32, 64);
    if (g4 == 0) sDgl[16 * it + r16] = dot * fexp2(gl_i);
#pragma unroll
    for (int kb = 0; kb < VB; ++kb)
#pragma unroll
      for (int tl = 0; tl < 4; ++tl) {
        uint4 xh, xl;
        afragx<LD>(sD + tl * RB, kb, lane, xh, xl);
        aK[tl] = mmx<LDH, LD>(fh[kb], fl[kb], xh, xl, aK[tl]);
      }
  }
  // dM tiles (c-block I, s-block J) = lower(dO delta^T) for lower tiles w and w + 8: mt lane -> column
  // s = 16 J + r16, rows c = 16 I + 4 g4 + j; mtT the same tile transposed, lane -> row c = 16 I + r16,
  // columns s = 16 J + 4 g4 + j.  Each gives one of the gradient phase's fragment forms directly.
  f32x4 mt[2], mtT[2];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    mt[x] = mtT[x] = zero4();
    const int t = w + NW * x;
    if (t >= 10) continue;
    int I, J;
    lower_tile(t, I, J);
#pragma unroll
    for (int kb = 0; kb < VB; ++kb) {
      uint4 xh, xl, oh, ol;
      afragx<LD>(sD + J * RB, kb, lane, xh, xl);
      afragx<LO_>(sO + I * RB, kb, lane, oh, ol);
      mt[x] = mmx<LO_, LD>(oh, ol, xh, xl, mt[x]);
      mtT[x] = mmx<LD, LO_>(xh, xl, oh, ol, mtT[x]);
    }
    if (I == J) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (r16 > 4 * g4 + j) mt[x][j] = 0.f;
        if (4 * g4 + j > r16) mtT[x][j] = 0.f;
      }
    }
  }

  if (flagged) {  // the exact kernels take it from here: store the products in their layouts
    __syncthreads();  // sDgl
    if (own_k) {
      const bufrsrc rQ = make_buf(xQg + ((int64_t)bh * T + t0) * K, L * K * 4);
      const bufrsrc rW = make_buf(xW + ((int64_t)bh * T + t0) * K, L * K * 4);
      const bufrsrc rKf = make_buf(xKf + ((int64_t)bh * T + t0) * K, L * K * 4);
#pragma unroll
      for (int tl = 0; tl < 4; ++tl) {
        const uint32_t c = (uint32_t)(16 * tl + r16);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, aQ[tl]), rQ, (c * K + i0) * 4, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, aK[tl]), rKf, (c * K + i0) * 4, 0, 0);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          buf_st(rW, ((uint32_t)(16 * tl + 4 * g4 + j) * K + 16 * it + r16) * 4, -aW[tl][j]);
      }
      if (g4 == 0) xgl[chunk * K + 16 * it + r16] = sDgl[16 * it + r16];
    }
    float* Mn = xM + chunk * C * C;
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const int t = w + NW * x;
      if (t >= 10) continue;
      int I, J;
      lower_tile(t, I, J);
#pragma unroll
      for (int j = 0; j < 4; ++j) Mn[(16 * I + 4 * g4 + j) * C + 16 * J + r16] = mt[x][j];
    }
    if (w < 6) {  // upper tiles are zero
      int I, J;
      upper_tile(w, I, J);
#pragma unroll
      for (int j = 0; j < 4; ++j) Mn[(16 * I + 4 * g4 + j) * C + 16 * J + r16] = 0.f;
    }
    return;
  }
  __syncthreads();  // phase-1 fragments dead: A^T may overwrite them
#pragma unroll
  for (int u = 0; u < AU; ++u) {
    const int e4 = tid + 512 * u, sr = e4 / (C / 4), c4 = e4 % (C / 4);
    *reinterpret_cast<float4*>(sAt + sr * AP4 + 4 * c4) = at_r[u];
  }
  __syncthreads();

  // ================================ solve ================================
  // Yt[0] = d delta^T A (V tile w), Yt[1] = dW^T A (K tile w); k = chunk row c in permuted order:
  // slot j of lane group g4 <-> c = 32 kb + 4 g4 + j (j < 4) or 32 kb + 16 + 4 g4 + (j - 4)
  const bufrsrc rdv = make_buf(dv + (((int64_t)b * T + t0) * H + h) * V, ((L - 1) * H + 1) * V * 2);
  f32x4 Yt[2][4];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int J = 0; J < 4; ++J) Yt[ct][J] = zero4();
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    uint4 xh0, xl0, xh1, xl1;
    {
      // d delta from phase 1's staged fragments (still intact: the partials overwrite them only after the barrier
      // that ends the solve's reads): element (c, v) of the [rows c][k = v] fragments, its bf16 hi and lo halves,
      // the split of the same value this column needs (a bf16 copy has no lo half)
      const uint16_t* f16 = reinterpret_cast<const uint16_t*>(sdD);
      const int v = 16 * w + r16;
      uint32_t xr[8], xq[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int c = 32 * kb + (j < 4 ? 4 * g4 + j : 16 + 4 * g4 + j - 4);
        const int off = (c >> 4) * RB + (v >> 5) * TILE + ((c & 15) + 16 * ((v & 31) >> 3)) * 8 + (v & 7);
        xr[j] = own_v ? (uint32_t)f16[off] : 0u;
        xq[j] = own_v && LDD ? (uint32_t)f16[off + 512] : 0u;
      }
      xh0 = uint4{xr[0] | (xr[1] << 16), xr[2] | (xr[3] << 16), xr[4] | (xr[5] << 16), xr[6] | (xr[7] << 16)};
      xl0 = uint4{xq[0] | (xq[1] << 16), xq[2] | (xq[3] << 16), xq[4] | (xq[5] << 16), xq[6] | (xq[7] << 16)};
    }
    {
      const f32x4 t0_ = -aW[2 * kb], t1_ = -aW[2 * kb + 1];  // zero for waves without a channel tile
      kdn_state::bfrag(t0_, t1_, xh1, xl1);
    }
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      if (J > 2 * kb + 1) continue;  // A[c][s] = 0 for c < s
      const float* row = sAt + (16 * J + r16) * AP4 + 32 * kb + 4 * g4;
      const float4 a0 = *reinterpret_cast<const float4*>(row), a1 = *reinterpret_cast<const float4*>(row + 16);
      const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
      uint4 ah, al;
      split8(av, ah, al);
      Yt[0][J] = mmx<LDD, true>(xh0, xl0, ah, al, Yt[0][J]);
      Yt[1][J] = mma3(xh1, xl1, ah, al, Yt[1][J]);
    }
  }
  if (own_v) {  // dv rows s = 16 J + r16, columns 16 w + 4 g4 .. + 3
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      const uint32_t tr = (uint32_t)(16 * J + r16), x0 = (uint32_t)(16 * w + 4 * g4);
      const f32x4 y = Yt[0][J];
      const uint32_t lo = (uint32_t)f2bf(y[0]) | ((uint32_t)f2bf(y[1]) << 16);
      const uint32_t hi = (uint32_t)f2bf(y[2]) | ((uint32_t)f2bf(y[3]) << 16);
      __builtin_amdgcn_raw_buffer_store_b64(u32x2{lo, hi}, rdv, ((tr * H) * V + x0) * 2, 0, 0);
    }
  }
  // this block's share of dN^T[s][c] = sum_x (U|W)[s][x] Y[x][c] (part: D tiles rows s, cols c) and the
  // same products transposed (part2: rows c, cols s), for the two orientations of the dN fragments
  f32x4 part[10], part2[10];
  {
    uint4 uh[4], ul[4], yh[4], yl[4];
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      const float4 a0 = uw[J][0], a1 = uw[J][1];
      const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
      split8(av, uh[J], ul[J]);
      kdn_state::bfrag(Yt[0][J], Yt[1][J], yh[J], yl[J]);
    }
#pragma unroll
    for (int t = 0; t < 10; ++t) {
      int I, J;
      lower_tile(t, I, J);
      part[t] = mma3(uh[J], ul[J], yh[I], yl[I], zero4());
      part2[t] = mma3(yh[I], yl[I], uh[J], ul[J], zero4());
    }
  }
  f32x4 kg[4];  // dKg^T tiles: lane -> chunk row 16 J + r16, channels i0 .. i0 + 3
#pragma unroll
  for (int J = 0; J < 4; ++J) kg[J] = Yt[1][J];
  __syncthreads();  // every A^T read done: the partials may overwrite it
  if (w >= 4) {
#pragma unroll
    for (int t = 0; t < 10; ++t) {
      *reinterpret_cast<f32x4*>(sP + (((w - 4) * 10 + t) * 64 + lane) * 4) = part[t];
      *reinterpret_cast<f32x4*>(sP2 + (((w - 4) * 10 + t) * 64 + lane) * 4) = part2[t];
    }
  }
  __syncthreads();
  if (w < 4) {
#pragma unroll
    for (int t = 0; t < 10; ++t) {
      f32x4* slot = reinterpret_cast<f32x4*>(sP + ((w * 10 + t) * 64 + lane) * 4);
      *slot = *slot + part[t];
      f32x4* slot2 = reinterpret_cast<f32x4*>(sP2 + ((w * 10 + t) * 64 + lane) * 4);
      *slot2 = *slot2 + part2[t];
    }
  }
  __syncthreads();

  // ======================= dN, dM staging (the gradient phase's fragments) =======================
  // fragment offset of 4 consecutive k = k0 .. k0 + 3 (k0 % 4 == 0) of one row: permuted k order, slot
  // 4 hh + j of lane group gg <-> k = 32 kb + 16 hh + 4 gg + j
  auto foff = [](int row, int k0) {
    return ((row >> 4) * 2 + (k0 >> 5)) * TILE + ((row & 15) + 16 * ((k0 & 15) >> 2)) * 8 + 4 * ((k0 >> 4) & 1);
  };
  // dN[c][s] = -(sum of the waves' partials), strictly lower: units (row, k0) of the rows form (row c,
  // k = s, from the part D tiles) and of the transposed form (row s, k = c, from the part2 D tiles)
  float4 dNu[2], dNtu[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int e = tid + 512 * u, row = e >> 4, kb = (e >> 3) & 1, hh = (e >> 2) & 1, gg = e & 3;
    const int k0 = 32 * kb + 16 * hh + 4 * gg;
    float4 acc = float4{0.f, 0.f, 0.f, 0.f}, acct = float4{0.f, 0.f, 0.f, 0.f};
    if ((k0 >> 4) <= (row >> 4)) {  // rows form: tile (c-block row / 16, s-block k0 / 16)
      const int t = lower_tile_index(row >> 4, k0 >> 4), ln = (row & 15) + 16 * ((k0 & 15) >> 2);
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) {
        const float4 v = *reinterpret_cast<const float4*>(sP + ((ww * 10 + t) * 64 + ln) * 4);
        acc.x -= v.x, acc.y -= v.y, acc.z -= v.z, acc.w -= v.w;
      }
      if (k0 + 0 >= row) acc.x = 0.f;
      if (k0 + 1 >= row) acc.y = 0.f;
      if (k0 + 2 >= row) acc.z = 0.f;
      if (k0 + 3 >= row) acc.w = 0.f;
    }
    if ((k0 >> 4) >= (row >> 4)) {  // transposed form: tile (c-block k0 / 16, s-block row / 16)
      const int t = lower_tile_index(k0 >> 4, row >> 4), ln = (row & 15) + 16 * ((k0 & 15) >> 2);
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) {
        const float4 v = *reinterpret_cast<const float4*>(sP2 + ((ww * 10 + t) * 64 + ln) * 4);
        acct.x -= v.x, acct.y -= v.y, acct.z -= v.z, acct.w -= v.w;
      }
      if (k0 + 0 <= row) acct.x = 0.f;
      if (k0 + 1 <= row) acct.y = 0.f;
      if (k0 + 2 <= row) acct.z = 0.f;
      if (k0 + 3 <= row) acct.w = 0.f;
    }
    dNu[u] = acc;
    dNtu[u] = acct;
  }
  __syncthreads();  // every partial read before the fragments overwrite them
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int e = tid + 512 * u, row = e >> 4, kb = (e >> 3) & 1, hh = (e >> 2) & 1, gg = e & 3;
    const int off = foff(row, 32 * kb + 16 * hh + 4 * gg);
    kdn_state::put_unit(sF, off, dNu[u].x, dNu[u].y, dNu[u].z, dNu[u].w);
    kdn_state::put_unit(sF + 2 * FR, off, dNtu[u].x, dNtu[u].y, dNtu[u].z, dNtu[u].w);
  }
#pragma unroll
  for (int x = 0; x < 2; ++x) {  // dM rows (row c, k = s) from mtT, dM^T rows (row s, k = c) from mt
    const int t = w + NW * x;
    if (t >= 16) continue;
    int I, J;
    f32x4 a = zero4(), at = zero4();
    if (t < 10) {
      lower_tile(t, I, J);
      a = mtT[x];
      at = mt[x];
    } else {
      upper_tile(t - 10, I, J);  // I < J: zero tiles of both forms
    }
    kdn_state::put_unit(sF + FR, foff(16 * I + r16, 16 * J + 4 * g4), a[0], a[1], a[2], a[3]);
    kdn_state::put_unit(sF + 3 * FR, foff(16 * J + r16, 16 * I + 4 * g4), at[0], at[1], at[2], at[3]);
  }
  if constexpr (QK_LDS || G_LDS) __builtin_amdgcn_s_waitcnt(0);  // this wave's k, q or G rows have reached LDS
  __syncthreads();

  // ================================ gradient phase ================================
  // With the in-op L2 norm (q_rstd, k_rstd [B,T,H] given) q and k are the raw inputs x, the operand is
  // y = bf16(x rstd) (the forward's), and dq, dk are returned for x: dx = rstd (dy - y (y . dy)), the
  // row dot summed over the waves.
  const bool qk_norm = q_rstd != nullptr;
  float bpart[4] = {0.f, 0.f, 0.f, 0.f};  // iso: dbeta partials of rows 16 tl + r16
  float dqs[4][4], dks[4][4];             // in-op norm: dy of q, k (rows 16 tl + r16, channels i0 ..)
  u32x2 yq2[4], yk2[4];                   // ... and y (bf16 pairs)
  if (own_k) {
    const bufrsrc rG = make_buf(gc + in_row0 * K, rows_in * K * 4);
    const bufrsrc rk = make_buf(k + in_row0 * K, rows_in * K * 2);
    const bufrsrc rq = make_buf(q + in_row0 * K, rows_in * K * 2);
    const bufrsrc rkap = ISO ? make_buf(kap + in_row0, rows_in * 4) : make_buf(kap + in_row0 * K, rows_in * K * 4);
    const bufrsrc rdq = make_buf(dq + in_row0 * K, rows_in * K * 2);
    const bufrsrc rdk = make_buf(dk + in_row0 * K, rows_in * K * 2);
    const bufrsrc rdkap = ISO ? make_buf(dkap, 0) : make_buf(dkap + in_row0 * K, rows_in * K * 4);
    const bufrsrc rdg = make_buf(dg + in_row0 * K, rows_in * K * 4);
    const int i = 16 * it + r16;
    // ---- factor loads, one channel per lane: rows c = 16 tl + 4 g4 + j, slot p = 4 tl + j; the gate
    // of rows past L repeats row L-1 (their k, q, kappa read zero)
    float av[16], Gv[16];
    uint16_t kraw[16], qraw[16];
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      const int c = 16 * (p >> 2) + 4 * g4 + (p & 3);
      const uint32_t crow = (uint32_t)(c * H), o = crow * K + i;
      if constexpr (QK_LDS) {
        kraw[p] = *reinterpret_cast<const uint16_t*>(qk_lds(0, c, i));
        qraw[p] = *reinterpret_cast<const uint16_t*>(qk_lds(1, c, i));
      } else {
        kraw[p] = __builtin_amdgcn_raw_buffer_load_b16(rk, o * 2, 0, 0);
        qraw[p] = __builtin_amdgcn_raw_buffer_load_b16(rq, o * 2, 0, 0);
      }
      av[p] = ISO ? sBt[ISO ? c : 0] : buf_ld(rkap, o * 4);
      if constexpr (G_LDS) Gv[p] = *g_lds(min(c, L - 1), i);
      else Gv[p] = buf_ld(rG, ((uint32_t)(min(c, L - 1) * H) * K + i) * 4);
    }
    __builtin_amdgcn_sched_barrier(0);
    float mA[4];  // block anchors m_J = (G_{16J} + G_{16J+15}) / 2 of this lane's channel
#pragma unroll
    for (int J = 0; J < 4; ++J) mA[J] = 0.5f * (__shfl(Gv[4 * J], r16, 64) + __shfl(Gv[4 * J + 3], 48 + r16, 64));
    float Rown[16], Kown[16], Qown[16];
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      const int c = 16 * (p >> 2) + 4 * g4 + (p & 3);
      float kvp = bf2f(kraw[p]), qvp = bf2f(qraw[p]);
      if (qk_norm) {
        kvp = l2n(kvp, sRs[1][c]);
        qvp = l2n(qvp, sRs[0][c]);
      }
      const float e = fexp2(Gv[p] - mA[p >> 2]);
      Kown[p] = kvp * e;
      Qown[p] = scale * qvp * e;
      Rown[p] = (ISO ? av[p] * kvp : av[p]) * frcp(e);
    }
    const float4 glv = G_LDS ? *reinterpret_cast<const float4*>(g_lds(L - 1, i0))
                             : buf_ld4(rG, ((uint32_t)((L - 1) * H) * K + i0) * 4);
    u32x2 kq4[4], qq4[4];
    float4 kap4[4], G4[4];
#pragma unroll
    for (int tl = 0; tl < 4; ++tl) {
      const uint32_t c = (uint32_t)(16 * tl + r16), o = c * H * K + i0;
      if constexpr (QK_LDS) {
        kq4[tl] = *reinterpret_cast<const u32x2*>(qk_lds(0, (int)c, i0));
        qq4[tl] = *reinterpret_cast<const u32x2*>(qk_lds(1, (int)c, i0));
      } else {
        kq4[tl] = __builtin_amdgcn_raw_buffer_load_b64(rk, o * 2, 0, 0);
        qq4[tl] = __builtin_amdgcn_raw_buffer_load_b64(rq, o * 2, 0, 0);
      }
      if (ISO) {
        const float be = sBt[ISO ? c : 0];
        kap4[tl] = float4{be, be, be, be};
      } else {
        kap4[tl] = buf_ld4(rkap, o * 4);
      }
      G4[tl] = G_LDS ? *reinterpret_cast<const float4*>(g_lds(min(16 * tl + r16, L - 1), i0))
                     : buf_ld4(rG, ((uint32_t)(min(16 * tl + r16, L - 1) * H) * K + i0) * 4);
    }
    float colpart[4] = {0.f, 0.f, 0.f, 0.f};
    float4 dg_last = float4{0.f, 0.f, 0.f, 0.f};
    bool has_last = false;
    const float gla[4] = {glv.x, glv.y, glv.z, glv.w};
#pragma unroll
    for (int tl = 0; tl < 4; ++tl) {
      f32x4 dLk = zero4(), dLq = zero4(), dR = zero4();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        uint4 ah, al;
        if (kb <= tl / 2) {
          const float s0 = 2 * kb <= tl ? fexp2(mA[tl] - mA[2 * kb]) : 0.f;
          const float s1 = 2 * kb + 1 <= tl ? fexp2(mA[tl] - mA[2 * kb + 1]) : 0.f;
          float rv[8];
#pragma unroll
          for (int sl = 0; sl < 8; ++sl) rv[sl] = Rown[8 * kb + sl] * (sl < 4 ? s0 : s1);
          uint4 Rh, Rl;
          split8(rv, Rh, Rl);
          afrag(sF, tl * 2 + kb, lane, ah, al);
          dLk = mma3(Rh, Rl, ah, al, dLk);
          afrag(sF + FR, tl * 2 + kb, lane, ah, al);
          dLq = mma3(Rh, Rl, ah, al, dLq);
        }
        if (2 * kb + 1 >= tl) {
          const float s0 = 2 * kb >= tl ? fexp2(mA[2 * kb] - mA[tl]) : 0.f;
          const float s1 = 2 * kb + 1 >= tl ? fexp2(mA[2 * kb + 1] - mA[tl]) : 0.f;
          float lk[8], lq[8];
#pragma unroll
          for (int sl = 0; sl < 8; ++sl) {
            const float sc = sl < 4 ? s0 : s1;
            lk[sl] = Kown[8 * kb + sl] * sc;
            lq[sl] = Qown[8 * kb + sl] * sc;
          }
          uint4 Kh, Kl, Qh, Ql;
          split8(lk, Kh, Kl);
          split8(lq, Qh, Ql);
          afrag(sF + 2 * FR, tl * 2 + kb, lane, ah, al);
          dR = mma3(Kh, Kl, ah, al, dR);
          afrag(sF + 3 * FR, tl * 2 + kb, lane, ah, al);
          dR = mma3(Qh, Ql, ah, al, dR);
        }
      }
      const uint32_t c = (uint32_t)(16 * tl + r16), o = c * H * K + i0;
      float kv4[4] = {__uint_as_float(kq4[tl].x << 16), __uint_as_float(kq4[tl].x & 0xffff0000u),
                      __uint_as_float(kq4[tl].y << 16), __uint_as_float(kq4[tl].y & 0xffff0000u)};
      float qv4[4] = {__uint_as_float(qq4[tl].x << 16), __uint_as_float(qq4[tl].x & 0xffff0000u),
                      __uint_as_float(qq4[tl].y << 16), __uint_as_float(qq4[tl].y & 0xffff0000u)};
      if (qk_norm) {
        const float rk_ = sRs[1][c], rq_ = sRs[0][c];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          kv4[j] = l2n(kv4[j], rk_);
          qv4[j] = l2n(qv4[j], rq_);
        }
        yk2[tl] = u32x2{(uint32_t)f2bf(kv4[0]) | ((uint32_t)f2bf(kv4[1]) << 16),
                        (uint32_t)f2bf(kv4[2]) | ((uint32_t)f2bf(kv4[3]) << 16)};  // exact: already bf16
        yq2[tl] = u32x2{(uint32_t)f2bf(qv4[0]) | ((uint32_t)f2bf(qv4[1]) << 16),
                        (uint32_t)f2bf(qv4[2]) | ((uint32_t)f2bf(qv4[3]) << 16)};
      }
      const float a4[4] = {kap4[tl].x, kap4[tl].y, kap4[tl].z, kap4[tl].w};
      const float gv[4] = {G4[tl].x, G4[tl].y, G4[tl].z, G4[tl].w};
      const float mz[4] = {__shfl(mA[tl], 4 * g4, 64), __shfl(mA[tl], 4 * g4 + 1, 64), __shfl(mA[tl], 4 * g4 + 2, 64),
                           __shfl(mA[tl], 4 * g4 + 3, 64)};
      float dkv[4], dqv[4], dav[4], dgv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float beta = ISO ? a4[j] : 0.f;
        const float kap_p = ISO ? beta * kv4[j] : a4[j];
        const float e = fexp2(gv[j] - mz[j]), er = frcp(e);
        const float eg = fexp2(gv[j]), f = fexp2(gla[j] - gv[j]);
        const float a_lk = dLk[j], a_lq = dLq[j] * scale, a_r = dR[j];
        const float dkgv = kg[tl][j], dqgv = aQ[tl][j], dkfv = aK[tl][j];
        dkv[j] = a_lk * e + dkgv * eg;
        dqv[j] = a_lq * e + scale * dqgv * eg;
        dav[j] = a_r * er + dkfv * f;
        dgv[j] = kv4[j] * e * a_lk + qv4[j] * e * a_lq - kap_p * er * a_r + kv4[j] * eg * dkgv +
                 scale * qv4[j] * eg * dqgv - kap_p * f * dkfv;
        if ((int)c < L) colpart[j] += kap_p * f * dkfv;
        if (ISO) {
          dkv[j] += beta * dav[j];
          bpart[tl] += dav[j] * kv4[j];
        }
      }
      if (!ISO)
        __builtin_amdgcn_raw_buffer_store_b128(
            u32x4{__float_as_uint(dav[0]), __float_as_uint(dav[1]), __float_as_uint(dav[2]), __float_as_uint(dav[3])},
            rdkap, o * 4, 0, 0);
      if (qk_norm) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          dqs[tl][j] = dqv[j];
          dks[tl][j] = dkv[j];
        }
      } else {
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{(uint32_t)f2bf(dqv[0]) | ((uint32_t)f2bf(dqv[1]) << 16),
                                                    (uint32_t)f2bf(dqv[2]) | ((uint32_t)f2bf(dqv[3]) << 16)},
                                              rdq, o * 2, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{(uint32_t)f2bf(dkv[0]) | ((uint32_t)f2bf(dkv[1]) << 16),
                                                    (uint32_t)f2bf(dkv[2]) | ((uint32_t)f2bf(dkv[3]) << 16)},
                                              rdk, o * 2, 0, 0);
      }
      if ((int)c == L - 1) {
        dg_last = float4{dgv[0], dgv[1], dgv[2], dgv[3]};
        has_last = true;
      } else {
        __builtin_amdgcn_raw_buffer_store_b128(
            u32x4{__float_as_uint(dgv[0]), __float_as_uint(dgv[1]), __float_as_uint(dgv[2]), __float_as_uint(dgv[3])},
            rdg, o * 4, 0, 0);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) colpart[j] = row16_sum(colpart[j]);
    if (has_last) {
      const float4 gl4 = *reinterpret_cast<const float4*>(sDgl + i0);
      const float4 v = float4{dg_last.x + colpart[0] + gl4.x, dg_last.y + colpart[1] + gl4.y,
                              dg_last.z + colpart[2] + gl4.z, dg_last.w + colpart[3] + gl4.w};
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rdg,
                                             ((uint32_t)((L - 1) * H) * K + i0) * 4, 0, 0);
    }
  }
  if (!ISO && !qk_norm) return;
  auto unpack4 = [](u32x2 v, float* f) {
    f[0] = __uint_as_float(v.x << 16), f[1] = __uint_as_float(v.x & 0xffff0000u);
    f[2] = __uint_as_float(v.y << 16), f[3] = __uint_as_float(v.y & 0xffff0000u);
  };
  if (own_k) {  // per-wave partials over this wave's 16 channels of rows 16 tl + r16
#pragma unroll
    for (int tl = 0; tl < 4; ++tl) {
      float v = bpart[tl], pq = 0.f, pk = 0.f;
      if (qk_norm) {
        float yq[4], yk[4];
        unpack4(yq2[tl], yq);
        unpack4(yk2[tl], yk);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          pq += yq[j] * dqs[tl][j];
          pk += yk[j] * dks[tl][j];
        }
      }
      v = swz16_add(v);
      pq = swz16_add(pq);
      pk = swz16_add(pk);
      v += __shfl_xor(v, 32, 64);
      pq += __shfl_xor(pq, 32, 64);
      pk += __shfl_xor(pk, 32, 64);
      if (g4 == 0) {
        sBeta[w * C + 16 * tl + r16] = v;
        sDot[0][w][16 * tl + r16] = pq;
        sDot[1][w][16 * tl + r16] = pk;
      }
    }
  }
  __syncthreads();
  if (ISO && tid < L) {
    float s = 0.f;
#pragma unroll
    for (int ww = 0; ww < NIT; ++ww) s += sBeta[ww * C + tid];
    dbeta[((int64_t)b * T + t0 + tid) * H + h] = s;
  }
  if (!qk_norm) return;
  if (tid < 2 * C) {  // the row dots: sum of the waves' partials, into slot 0
    const int tq = tid >> 6, c = tid & 63;
    float dsum = 0.f;
#pragma unroll
    for (int ww = 0; ww < NIT; ++ww) dsum += sDot[tq][ww][c];
    sDot[tq][NW - 1][c] = dsum;  // each (tensor, row) is read and overwritten by this one thread
  }
  __syncthreads();
  if (own_k) {  // dx = rstd (dy - y (y . dy)) for the raw q, k
    const bufrsrc rdq = make_buf(dq + in_row0 * K, rows_in * K * 2);
    const bufrsrc rdk = make_buf(dk + in_row0 * K, rows_in * K * 2);
#pragma unroll
    for (int tl = 0; tl < 4; ++tl) {
      const int c = 16 * tl + r16;
      const float dotq = sDot[0][NW - 1][c], dotk = sDot[1][NW - 1][c];
      const float rq_ = sRs[0][c], rk_ = sRs[1][c];
      float yq[4], yk[4], xq[4], xk[4];
      unpack4(yq2[tl], yq);
      unpack4(yk2[tl], yk);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xq[j] = rq_ * (dqs[tl][j] - yq[j] * dotq);
        xk[j] = rk_ * (dks[tl][j] - yk[j] * dotk);
      }
      const uint32_t o = (uint32_t)(c * H) * K + i0;
      __builtin_amdgcn_raw_buffer_store_b64(u32x2{(uint32_t)f2bf(xq[0]) | ((uint32_t)f2bf(xq[1]) << 16),
                                                  (uint32_t)f2bf(xq[2]) | ((uint32_t)f2bf(xq[3]) << 16)},
                                            rdq, o * 2, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b64(u32x2{(uint32_t)f2bf(xk[0]) | ((uint32_t)f2bf(xk[1]) << 16),
                                                  (uint32_t)f2bf(xk[2]) | ((uint32_t)f2bf(xk[3]) << 16)},
                                            rdk, o * 2, 0, 0);
    }
  }
}

// One workgroup per task: tasks task0 .. task0 + gridDim.x - 1.
template <int K, int V, bool ISO, typename TDO, int HM>
__global__ __launch_bounds__(512, 1) void chunk_bwd_kernel(
    const void* __restrict__ hbuf, const void* __restrict__ dhbuf, const void* __restrict__ Dl,
    const void* __restrict__ dDl, const TDO* __restrict__ dO, const float* __restrict__ At,
    const float* __restrict__ U, const float* __restrict__ W, const int* __restrict__ flags,
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const float* __restrict__ kap,
    const float* __restrict__ gc, const float* __restrict__ q_rstd, const float* __restrict__ k_rstd, int T, int H,
    int NT, int BH, int task0, float scale, bf16_t* __restrict__ dv, bf16_t* __restrict__ dq, bf16_t* __restrict__ dk,
    float* __restrict__ dkap, float* __restrict__ dbeta, float* __restrict__ dg, float* __restrict__ xQg,
    float* __restrict__ xW, float* __restrict__ xKf, float* __restrict__ xM, float* __restrict__ xgl) {
  chunk_bwd_task<K, V, ISO, TDO, HM>(task0 + (int)blockIdx.x, hbuf, dhbuf, Dl, dDl, dO, At, U, W, flags, q, k, kap, gc,
                                 q_rstd, k_rstd, T, H, NT, BH, scale, dv, dq, dk, dkap, dbeta, dg, xQg, xW, xKf, xM,
                                 xgl);
}

}  // namespace kdn_bwd
