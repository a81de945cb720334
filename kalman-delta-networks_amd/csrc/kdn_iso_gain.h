// Isotropic Kalman gain (one scalar covariance per head): the map algebra, the kernels that the standalone
// gain entry points and the fused iso front share, and the per-chunk pieces that the fused front runs
// inside the gate's kernels.  Reference lit_gpt/kdn_ops/iso_kdn_chunk.py:1464-1893.
//
//   z = a p + w;  beta = z / (r + z);  p' = r z / (r + s z)    (s = info_scale / K)
//   forward map of a token:  p -> (r a p + r w) / (s a p + r + s w), a projective (Mobius) 2x2 map, so a
//                            token range composes into one map;
//   backward (reverse):      lambda_{t-1} = A_t lambda_t + B_t,
//                            A_t = a r^2 / (r + s z)^2,  B_t = a dbeta r / (r + z)^2, an affine map.
// a, omega, r, beta, p_prev are [B,T,H] (heads interleaved); the chunk is 64 tokens.  Chunk maps are
// [B*H][NC] (float4 forward, float2 backward).
#pragma once
#include "kdn_common.h"

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
// The same with the hardware reciprocal (v_rcp_f32, 1 ulp) instead of the IEEE division sequence: the
// isotropic gain's passes are chains of dependent map products, and a Mobius map is invariant under a
// common factor, so the renormalisation needs no exact reciprocal.
__device__ __forceinline__ Map2 map_mul_r(const Map2& a, const Map2& b) {
  Map2 c{a.m0 * b.m0 + a.m1 * b.m2, a.m0 * b.m1 + a.m1 * b.m3, a.m2 * b.m0 + a.m3 * b.m2,
         a.m2 * b.m1 + a.m3 * b.m3};
  const float s = fmaxf(fmaxf(fabsf(c.m0), fabsf(c.m1)), fmaxf(fabsf(c.m2), fabsf(c.m3)));
  const float inv = frcp(fmaxf(s, 1e-30f));
  c.m0 *= inv; c.m1 *= inv; c.m2 *= inv; c.m3 *= inv;
  return c;
}
__device__ __forceinline__ float mobius_r(const Map2& m, float p) { return (m.m0 * p + m.m1) * frcp(m.m2 * p + m.m3); }
__device__ __forceinline__ Map2 map_identity() { return Map2{1.f, 0.f, 0.f, 1.f}; }
__device__ __forceinline__ Map2 map_of(float4 m) { return Map2{m.x, m.y, m.z, m.w}; }
__device__ __forceinline__ Map2 token_map(float at, float wt, float rt, float s) {
  return Map2{rt * at, rt * wt, s * at, rt + s * wt};
}
__device__ __forceinline__ Map2 shfl_down_map(const Map2& m, int d) {
  return Map2{__shfl_down(m.m0, d, 64), __shfl_down(m.m1, d, 64), __shfl_down(m.m2, d, 64), __shfl_down(m.m3, d, 64)};
}

// Affine maps x -> A x + B of the reverse recurrence; compose(f, g) = f o g (g applied first).
__device__ __forceinline__ float2 aff_compose(float2 f, float2 g) { return float2{f.x * g.x, f.x * g.y + f.y}; }
__device__ __forceinline__ float2 token_aff(float at, float wt, float rt, float dl, float pp, float s) {
  const float z = at * pp + wt;
  const float ig = frcp(rt + z), ip = frcp(rt + s * z);
  return float2{at * rt * rt * ip * ip, at * dl * rt * ig * ig};
}
__device__ __forceinline__ float2 shfl_down_aff(float2 f, int d) {
  return float2{__shfl_down(f.x, d, 64), __shfl_down(f.y, d, 64)};
}

// The cotangents of one token's a, omega, r given lambda after the token (the cotangent of the covariance
// it passes on) and its beta cotangent dl; returns lambda before the token (a zbar).
__device__ __forceinline__ float token_grad(float at, float wt, float rt, float dl, float pp, float lam, float s,
                                            bool unit_scale, float& da, float& dw, float& dr) {
  const float z = at * pp + wt;
  const float ig = frcp(rt + z);
  const float ig2 = ig * ig;
  float zbar, drt;
  if (unit_scale) {
    zbar = (dl + rt * lam) * rt * ig2;
    drt = z * (lam * z - dl) * ig2;
  } else {
    const float ip = frcp(rt + s * z);
    const float ip2 = ip * ip;
    zbar = dl * rt * ig2 + lam * rt * rt * ip2;
    drt = -dl * z * ig2 + lam * s * z * z * ip2;
  }
  da = zbar * pp;
  dw = zbar;
  dr = drt;
  return at * zbar;
}

// ----------------------------------------------------------------------------
// Chunk kernels: one workgroup per (chunk, batch row) stages the chunk's contiguous [64][H] tiles in LDS;
// four threads per head compose or replay 16 tokens each.
// ----------------------------------------------------------------------------
constexpr int kIsoChunk = 64;
constexpr int kIsoSub = 4;  // threads per head in a chunk (16 tokens each)

// Stage rows [t0, t0 + L) of NA [B,T,H] arrays into NA consecutive LDS tiles tile[t][h] (coalesced;
// tile a at tiles + a * 64 * H).  A thread's loads of one round (kStageU elements of every array) all go
// out before the first LDS write: the element index is clamped into the tile, so the loads carry no
// branch and the thread waits for memory once per round instead of once per element.
constexpr int kStageU = 5;  // 5 * 256 threads cover a 64-token tile of up to 20 heads in one round
template <int NA>
__device__ __forceinline__ void stage_bth_n(const float* const (&x)[NA], int b, int T, int H, int t0, int L,
                                            float* tiles) {
  const int64_t base = ((int64_t)b * T + t0) * H;
  const int n = L * H;
  for (int e0 = threadIdx.x; e0 < n; e0 += kStageU * blockDim.x) {
    float v[kStageU][NA];
#pragma unroll
    for (int u = 0; u < kStageU; ++u) {
      const int64_t e = base + min(e0 + u * (int)blockDim.x, n - 1);
#pragma unroll
      for (int q = 0; q < NA; ++q) v[u][q] = x[q][e];
    }
#pragma unroll
    for (int u = 0; u < kStageU; ++u) {
      const int e = e0 + u * (int)blockDim.x;
      if (e < n) {
#pragma unroll
        for (int q = 0; q < NA; ++q) tiles[q * kIsoChunk * H + e] = v[u][q];
      }
    }
  }
}
__device__ __forceinline__ void store_bth(float* __restrict__ x, int b, int T, int H, int t0, int L,
                                          const float* tile) {
  const int64_t base = ((int64_t)b * T + t0) * H;
  for (int e = threadIdx.x; e < L * H; e += blockDim.x) x[base + e] = tile[e];
}

// The covariance at the start of an emit workgroup's chunk n comes from the chunk maps 0 .. n-1.
// carry_tph(H) consecutive lanes share a head; each composes a contiguous run of those chunks, and the
// runs are combined in order over the lane group.  With SM the first 64 chunk maps of every head are
// staged in LDS first (coalesced loads, issued with the token tiles' loads) in rows of 72 float4, chunk c
// at c + c / 8, so the 8 chunks a lane reads per step fall in distinct banks.
__device__ __forceinline__ int carry_tph(int H) {
  int tph = 64;  // lanes per head: a power of two, at most a wave, with tph * H <= 256 (H <= 96: tph >= 2)
  while (tph * H > 256) tph >>= 1;
  return tph;
}
constexpr int kMapRow = 72;  // float4 per head row of staged chunk maps (64 chunks + 8 pad)
__device__ __forceinline__ int map_slot(int c) { return c + (c >> 3); }
// Floats of the emit kernel's dynamic LDS: 5 token tiles, the sub-segment maps, the carries, then with SM
// (16-byte aligned) the staged maps.
__host__ __device__ inline int iso_emit_lds_floats(int H, bool sm) {
  const int base = (5 * kIsoChunk * H + 4 * kIsoSub * H + H + 3) & ~3;
  return base + (sm ? 4 * kMapRow * H : 0);
}

// grid (NC, B), block 256.  Workgroup (n, b) first finds the covariance at the start of its chunk for
// every head: p = (chunk maps 0 .. n-1)(1 / mu).  The initial precision mu is per head ([H], prec_mode 0)
// or per batch row and head ([B,H], prec_mode 1: the final precision of an earlier segment of the same
// sequences).  It then replays its tokens (beta, and the incoming covariance p_prev for the backward);
// the last chunk's workgroup also writes the final precision 1 / p_T.
template <bool SM>
__global__ __launch_bounds__(256) void iso_gain_emit_kernel(const float* __restrict__ a, const float* __restrict__ omega,
                                                            const float* __restrict__ r, const float4* __restrict__ maps,
                                                            const float* __restrict__ mu, int prec_mode, int T, int H,
                                                            int NC, float s, int unit_scale, float* __restrict__ beta,
                                                            float* __restrict__ p_prev,
                                                            float* __restrict__ final_precision) {
  extern __shared__ float sm[];
  float *sa = sm, *sw = sm + kIsoChunk * H, *sr = sm + 2 * kIsoChunk * H, *sbeta = sm + 3 * kIsoChunk * H,
        *spp = sm + 4 * kIsoChunk * H;
  Map2* sub = reinterpret_cast<Map2*>(sm + 5 * kIsoChunk * H);
  float* sCarry = sm + 5 * kIsoChunk * H + 4 * kIsoSub * H;
  float4* sMap = reinterpret_cast<float4*>(sm + iso_emit_lds_floats(H, false));
  const int n = blockIdx.x, b = blockIdx.y, t0 = n * kIsoChunk, L = min(kIsoChunk, T - t0);
  const int tph = carry_tph(H), hc = min((int)threadIdx.x / tph, H - 1), j = threadIdx.x % tph;
  const int64_t bhc = (int64_t)b * H + hc;
  const int cpt = (n + tph - 1) / tph, cA = j * cpt, cB = min(n, cA + cpt);  // this lane's chunks [cA, cB)
  const float muc = mu[prec_mode ? bhc : hc];
  const int ns = min(n, 64);  // chunks staged per head (SM)
  constexpr int MU = 5;
  float4 mv[MU];  // loads that go out with the token tiles': the first round of the map staging (SM) or
                  // this lane's first MU chunk maps
  if (SM) {
#pragma unroll
    for (int u = 0; u < MU; ++u) {
      const int e = min((int)threadIdx.x + u * (int)blockDim.x, max(H * ns - 1, 0));
      mv[u] = maps[((int64_t)b * H + e / max(ns, 1)) * NC + e % max(ns, 1)];
    }
  } else {
#pragma unroll
    for (int u = 0; u < MU; ++u) mv[u] = maps[bhc * NC + min(cA + u, max(n - 1, 0))];
  }
  stage_bth_n<3>({a, omega, r}, b, T, H, t0, L, sa);
  if (SM) {
#pragma unroll
    for (int u = 0; u < MU; ++u) {  // round 0 from the registers loaded above
      const int e = threadIdx.x + u * (int)blockDim.x;
      if (e < H * ns) sMap[(e / ns) * kMapRow + map_slot(e % ns)] = mv[u];
    }
    for (int e0 = threadIdx.x + MU * blockDim.x; e0 < H * ns; e0 += MU * blockDim.x) {  // H * ns > 1280 only
      float4 t5[MU];
#pragma unroll
      for (int u = 0; u < MU; ++u) {
        const int e = min(e0 + u * (int)blockDim.x, H * ns - 1);
        t5[u] = maps[((int64_t)b * H + e / ns) * NC + e % ns];
      }
#pragma unroll
      for (int u = 0; u < MU; ++u) {
        const int e = e0 + u * (int)blockDim.x;
        if (e < H * ns) sMap[(e / ns) * kMapRow + map_slot(e % ns)] = t5[u];
      }
    }
    __syncthreads();
  }
  {
    Map2 M = map_identity();
    if (SM) {
      for (int c = cA; c < cB; ++c)
        M = map_mul_r(map_of(c < 64 ? sMap[hc * kMapRow + map_slot(c)] : maps[bhc * NC + c]), M);
    } else {
#pragma unroll
      for (int u = 0; u < MU; ++u)
        if (cA + u < cB) M = map_mul_r(map_of(mv[u]), M);
      for (int c0 = cA + MU; c0 < cB; c0 += 8) {  // the rest in batches of 8 loads
        float4 t8[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) t8[u] = maps[bhc * NC + min(c0 + u, cB - 1)];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (c0 + u < cB) M = map_mul_r(map_of(t8[u]), M);
      }
    }
    for (int d = 1; d < tph; d <<= 1) {  // lane j takes lane j + d's composite (later chunks) as applied after its own
      const Map2 o = shfl_down_map(M, d);
      if ((j & (2 * d - 1)) == 0) M = map_mul_r(o, M);
    }
    if (j == 0 && (int)threadIdx.x / tph < H) sCarry[hc] = mobius_r(M, 1.f / muc);
  }
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
  for (int hq = threadIdx.x; hq < kIsoSub * H; hq += blockDim.x) {
    const int h = hq / kIsoSub, q = hq % kIsoSub;
    Map2 E = map_identity();
    for (int q2 = 0; q2 < q; ++q2) E = map_mul_r(sub[kIsoSub * h + q2], E);
    float p = mobius_r(E, sCarry[h]);
    for (int t = q * SL; t < min(L, (q + 1) * SL); ++t) {
      const float at = sa[t * H + h], wt = sw[t * H + h], rt = sr[t * H + h];
      spp[t * H + h] = p;
      const float z = at * p + wt;
      const float g = z * frcp(rt + z);
      sbeta[t * H + h] = g;
      p = unit_scale ? rt * g : rt * z * frcp(rt + s * z);
    }
    if (final_precision && n == NC - 1 && q == (L - 1) / SL) final_precision[(int64_t)b * H + h] = 1.f / p;
  }
  __syncthreads();
  store_bth(beta, b, T, H, t0, L, sbeta);
  if (p_prev) store_bth(p_prev, b, T, H, t0, L, spp);
}

// grid (NC, B), block 256, dynamic LDS 5 * 64 * H floats + 2 * 4 * H: the reverse chunk map of every
// head (lambda before the chunk from lambda after it).
__global__ __launch_bounds__(256) void iso_gain_bwd_map_kernel(const float* __restrict__ a,
                                                               const float* __restrict__ omega,
                                                               const float* __restrict__ r,
                                                               const float* __restrict__ dbeta,
                                                               const float* __restrict__ p_prev, int T, int H, int NC,
                                                               float s, float2* __restrict__ maps) {
  extern __shared__ float sm[];
  float *sa = sm, *sw = sm + kIsoChunk * H, *sr = sm + 2 * kIsoChunk * H, *sd = sm + 3 * kIsoChunk * H,
        *sp = sm + 4 * kIsoChunk * H;
  float2* sub = reinterpret_cast<float2*>(sm + 5 * kIsoChunk * H);
  const int n = blockIdx.x, b = blockIdx.y, t0 = n * kIsoChunk, L = min(kIsoChunk, T - t0);
  stage_bth_n<5>({a, omega, r, dbeta, p_prev}, b, T, H, t0, L, sa);
  __syncthreads();
  constexpr int SL = kIsoChunk / kIsoSub;
  for (int hq = threadIdx.x; hq < kIsoSub * H; hq += blockDim.x) {
    const int h = hq / kIsoSub, q = hq % kIsoSub;
    float2 F{1.f, 0.f};  // lambda before the sub-segment from lambda after it
    for (int t = min(L, (q + 1) * SL) - 1; t >= q * SL; --t) {
      const int e = t * H + h;
      F = aff_compose(token_aff(sa[e], sw[e], sr[e], sd[e], sp[e], s), F);  // earlier token applied after
    }
    sub[hq] = F;
  }
  __syncthreads();
  for (int h = threadIdx.x; h < H; h += blockDim.x) {
    float2 F = sub[kIsoSub * h + kIsoSub - 1];
    for (int q = kIsoSub - 2; q >= 0; --q) F = aff_compose(sub[kIsoSub * h + q], F);
    maps[((int64_t)b * H + h) * NC + n] = F;
  }
}

// Host launchers of the two shared kernels (grid (NC, B), block 256).  The emit stages the chunk maps in
// LDS when its dynamic LDS stays within 64 KB (H <= 26).
inline void launch_iso_gain_emit(const float* a, const float* omega, const float* r, const float4* maps,
                                 const float* mu, int prec_mode, int B, int T, int H, int NC, float s, float* beta,
                                 float* p_prev, float* final_precision, hipStream_t stream) {
  const int unit = s == 1.f ? 1 : 0;
  const bool stage = iso_emit_lds_floats(H, true) * sizeof(float) <= 64 * 1024;
  const size_t lds = (size_t)iso_emit_lds_floats(H, stage) * sizeof(float);
  if (stage)
    hipLaunchKernelGGL(iso_gain_emit_kernel<true>, dim3(NC, B), dim3(256), lds, stream, a, omega, r, maps, mu,
                       prec_mode, T, H, NC, s, unit, beta, p_prev, final_precision);
  else
    hipLaunchKernelGGL(iso_gain_emit_kernel<false>, dim3(NC, B), dim3(256), lds, stream, a, omega, r, maps, mu,
                       prec_mode, T, H, NC, s, unit, beta, p_prev, final_precision);
}
inline void launch_iso_gain_bwd_map(const float* a, const float* omega, const float* r, const float* dbeta,
                                    const float* p_prev, int B, int T, int H, int NC, float s, float2* maps,
                                    hipStream_t stream) {
  const size_t lds = (size_t)(5 * kIsoChunk * H + 2 * kIsoSub * H) * sizeof(float);
  hipLaunchKernelGGL(iso_gain_bwd_map_kernel, dim3(NC, B), dim3(256), lds, stream, a, omega, r, dbeta, p_prev, T, H,
                     NC, s, maps);
}

// ----------------------------------------------------------------------------
// Pieces of the gain that the fused front runs inside the gate's kernels, whose workgroups own one
// (batch row, 64-token chunk, head): lane t of wave 0 holds token t0 + t.
// ----------------------------------------------------------------------------

// The chunk's forward map from its tokens' maps (lane t: token t's map, the identity past the chunk's
// end): an ordered reduction over the wave; lane 0 returns the map of the whole chunk.
__device__ __forceinline__ Map2 wave_chunk_map(Map2 M) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const Map2 o = shfl_down_map(M, d);
    if ((lane & (2 * d - 1)) == 0) M = map_mul_r(o, M);  // lane + d holds later tokens: applied after
  }
  return M;
}

struct IsoGainBwdArgs {
  const float2* maps;                             // [B*H][NC] reverse chunk maps
  const float *a, *omega, *r, *dbeta, *p_prev;    // [B,T,H]
  const float* fprec;                             // [B,H] final precision (read with dfprec)
  const float* dfprec;                            // [B,H] its cotangent, nullable
  const float* mu;                                // initial precision: [H] (prec_mode 0) or [B,H]
  float* dmu_rows;  // -lambda_0 / mu^2 per (b, h) [B*H], nullable: per row of a per-head mu (summed later)
                    // for prec_mode 0, the [B,H] initial precision's cotangent for prec_mode 1
  int prec_mode, NC, unit_scale;
  float s;
};

// The gain's backward over chunk n of (b, h), run by wave 0 of a workgroup that owns it: lane t returns
// the cotangents of a, omega, r of token t0 + t (zero past the chunk's end).  Lambda after the chunk comes
// from lambda_T (the final precision's cotangent, -dc c_T^2) and the chunk maps NC-1 .. n+1 (64 per
// ordered wave reduction, the latest group first); lambda after each token from an inclusive suffix scan
// of the tokens' affine maps over the lanes.  Chunk 0's lane 0 also writes d mu = -lambda_0 / mu^2.
__device__ __forceinline__ void iso_gain_bwd_chunk(const IsoGainBwdArgs& G, int b, int n, int h, int T, int H,
                                                   int L, float& da, float& dw, float& dr) {
  const int lane = threadIdx.x & 63;
  const int64_t bh = (int64_t)b * H + h;
  const int64_t row = ((int64_t)b * T + (int64_t)n * kIsoChunk + min(lane, L - 1)) * H + h;
  // every load first: the latest group of later chunks, the token's inputs, lambda_T
  const int cl = G.NC - 64 + lane;
  float2 F = cl > n ? G.maps[bh * G.NC + cl] : float2{1.f, 0.f};
  const float at = G.a[row], wt = G.omega[row], rt = G.r[row], dl = G.dbeta[row], pp = G.p_prev[row];
  float lam = G.dfprec ? -G.dfprec[bh] * G.fprec[bh] * G.fprec[bh] : 0.f;
  for (int c1 = G.NC; c1 > n + 1; c1 -= 64) {
    if (c1 != G.NC) {
      const int c = c1 - 64 + lane;
      F = c > n ? G.maps[bh * G.NC + c] : float2{1.f, 0.f};
    }
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {  // lane + d holds later chunks: applied first
      const float2 o = shfl_down_aff(F, d);
      if ((lane & (2 * d - 1)) == 0) F = aff_compose(F, o);
    }
    lam = __shfl(F.x, 0, 64) * lam + __shfl(F.y, 0, 64);
  }
  // S_t = F_t o F_{t+1} o ... o F_63 (lambda before token t from lambda after the chunk)
  float2 S = lane < L ? token_aff(at, wt, rt, dl, pp, G.s) : float2{1.f, 0.f};
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const float2 o = shfl_down_aff(S, d);
    if (lane + d < 64) S = aff_compose(S, o);
  }
  float2 Sn = shfl_down_aff(S, 1);  // lambda after token t = S_{t+1}(lambda after the chunk)
  if (lane == 63) Sn = float2{1.f, 0.f};
  const float lam_t = Sn.x * lam + Sn.y;
  da = dw = dr = 0.f;
  if (lane < L) {
    const float lam_before = token_grad(at, wt, rt, dl, pp, lam_t, G.s, G.unit_scale != 0, da, dw, dr);
    if (G.dmu_rows && n == 0 && lane == 0) {
      const float m = G.mu[G.prec_mode ? bh : h];
      G.dmu_rows[bh] = -lam_before / (m * m);
    }
  }
}

}  // namespace
