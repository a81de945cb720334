// Serial chunk-state passes of the KDN memory scan (forward and reverse).
//
//   forward  (per chunk n):  h_n = S;  delta = U - W S;  O = Qg S + M delta;
//                            S = e^{g_last} S + Kf^T delta
//   backward (reverse):      dh_n = dS;  d delta = M^T dO + Kf dS;
//                            dS <- e^{g_last} dS + Qg^T dO - W^T d delta
//
// Work split.  One workgroup per (b, h, 64-column slice of V), one wave per 16 state columns;
// each wave keeps its columns for the whole sequence as K/16 MFMA accumulator tiles.  The
// workgroups of one (b, h) are placed on one XCD so the chunk operands they both read are
// shared through that XCD's L2.
//
// Precision.  Products use bf16x3 split MFMA (v_mfma_f32_16x16x32_bf16 on hi*hi + hi*lo +
// lo*hi of x = hi + lo, both halves rounded to nearest even), ~2^-16 relative per product with
// fp32 accumulation.  A bf16 output cotangent is exact in one half, so its products take two.
//
// Operand flow.
//  * B operands are the recurrent state and the chunk's delta, taken straight from the
//    accumulators.  The D layout of a 16x16 MFMA tile gives lane l the rows 4(l/16)+j of
//    column l%16, so two stacked row tiles supply the 8 k-values a 16x16x32 B fragment needs
//    once the k index is permuted inside each 32-block: slot s of lane group g = l/16 holds
//    k = 4g + s (s < 4) or 16 + 4g + (s - 4) (s >= 4).  The A fragments use the same order.
//  * A operands (chunk matrices shared by the 4 waves) are split to bf16 hi/lo once per
//    workgroup and stored in LDS in fragment order: a 16 x 32 tile is 64 lanes x 8 bf16 of hi
//    followed by the same for lo, so a fragment is one contiguous 16-byte read per lane.
//  * Each chunk update has two phases with an LDS buffer each.  While a phase multiplies out
//    of its buffer, the threads split the other phase's next operands (loaded into registers
//    one phase earlier) into the other buffer: two barriers per chunk, loads one phase ahead.
#pragma once
#include <type_traits>
#include "kdn_common.h"

namespace kdn_state {

constexpr int C = 64;
// V columns per workgroup (16 per wave).  64 columns (4 waves) keeps twice as many CUs busy as
// one 128-column workgroup per (b, h), which measures faster: the pass is bound by each CU's
// chunk-operand throughput, not by the duplicated operand splitting.
__host__ __device__ constexpr int state_cols(int V) { return V < 64 ? V : 64; }
__host__ __device__ constexpr int state_threads(int V) { return 4 * state_cols(V); }
constexpr int TILE = 1024;   // bf16 elements of one 16 x 32 A tile (hi 512, lo 512)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4 mfma(uint4 a, uint4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}
// a*b with a = ah + al, b = bh + bl, dropping al*bl
__device__ __forceinline__ f32x4 mma3(uint4 ah, uint4 al, uint4 bh, uint4 bl, f32x4 c) {
  c = mfma(ah, bh, c);
  c = mfma(ah, bl, c);
  c = mfma(al, bh, c);
  return c;
}
// a*b with b exact in bf16
__device__ __forceinline__ f32x4 mma2(uint4 ah, uint4 al, uint4 b, f32x4 c) {
  c = mfma(ah, b, c);
  c = mfma(al, b, c);
  return c;
}
__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Two floats -> packed bf16 (RNE), element 0 in the low half.
__device__ __forceinline__ uint32_t pk2(float a, float b) {
  bf16x2v v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ void split2(float a, float b, uint32_t& hi, uint32_t& lo) {
  hi = pk2(a, b);
  lo = pk2(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xffff0000u));
}
// 4 x 4 transpose across a lane quad: lane r of the quad holds row r (x, y, z, w = columns 0..3)
// on entry and column r (rows 0..3) on return.  Two butterfly stages with DPP quad permutations:
// swap the off-diagonal elements of the 2 x 2 blocks between lanes r and r ^ 1, then the
// off-diagonal 2 x 2 blocks between lanes r and r ^ 2.
__device__ __forceinline__ float4 quad_transpose(const float4& x, int r) {
  auto dpp = [](float v, int ctrl) {
    return __int_as_float(ctrl == 0xb1 ? __builtin_amdgcn_mov_dpp(__float_as_int(v), 0xb1, 0xf, 0xf, false)
                                       : __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4e, 0xf, 0xf, false));
  };
  float a0 = x.x, a1 = x.y, a2 = x.z, a3 = x.w;
  const bool odd = r & 1, hi = r & 2;
  {  // lanes r, r ^ 1: even lanes take the partner's columns 0, 2 into slots 1, 3; odd lanes the reverse
    const float r0 = dpp(odd ? a0 : a1, 0xb1), r1 = dpp(odd ? a2 : a3, 0xb1);
    a0 = odd ? r0 : a0;
    a1 = odd ? a1 : r0;
    a2 = odd ? r1 : a2;
    a3 = odd ? a3 : r1;
  }
  {  // lanes r, r ^ 2: the upper lanes take the partner's slots 2, 3 into slots 0, 1; lower the reverse
    const float r0 = dpp(hi ? a0 : a2, 0x4e), r1 = dpp(hi ? a1 : a3, 0x4e);
    a0 = hi ? r0 : a0;
    a1 = hi ? r1 : a1;
    a2 = hi ? a2 : r0;
    a3 = hi ? a3 : r1;
  }
  return float4{a0, a1, a2, a3};
}
// Orders one wave's LDS accesses around a cross-lane exchange: the LDS unit serves a wave's
// instructions in issue order, so only the compiler's reordering has to be fenced off.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
// 8 floats -> split hi/lo fragment (slot j <- x[j])
__device__ __forceinline__ void split8v(const float* x, uint4& hi, uint4& lo) {
  split2(x[0], x[1], hi.x, lo.x);
  split2(x[2], x[3], hi.y, lo.y);
  split2(x[4], x[5], hi.z, lo.z);
  split2(x[6], x[7], hi.w, lo.w);
}
// hi/lo B fragment from two stacked D-layout tiles (k rows [0,16) and [16,32) of a block).
__device__ __forceinline__ void bfrag(f32x4 t0, f32x4 t1, uint4& hi, uint4& lo) {
  split2(t0[0], t0[1], hi.x, lo.x);
  split2(t0[2], t0[3], hi.y, lo.y);
  split2(t1[0], t1[1], hi.z, lo.z);
  split2(t1[2], t1[3], hi.w, lo.w);
}

// Staging unit u of an A operand with contraction length KD: 4 consecutive k-slots of one lane
// of one tile.  Consecutive u are consecutive lanes, so a wave's LDS stores are contiguous.
struct Unit {
  int row, k0, off;
};
template <int KD>
__device__ __forceinline__ Unit unit(int u) {
  constexpr int KB = KD / 32;
  const int tile = u >> 7, half = (u >> 6) & 1, L = u & 63;
  return Unit{16 * (tile / KB) + (L & 15), 32 * (tile % KB) + 16 * half + 4 * (L >> 4), tile * TILE + L * 8 + 4 * half};
}
__device__ __forceinline__ void put_unit(bf16_t* buf, int off, float a, float b, float c, float d) {
  uint32_t h0, l0, h1, l1;
  split2(a, b, h0, l0);
  split2(c, d, h1, l1);
  *reinterpret_cast<uint2*>(buf + off) = uint2{h0, h1};
  *reinterpret_cast<uint2*>(buf + off + 512) = uint2{l0, l1};
}
__device__ __forceinline__ void afrag(const bf16_t* buf, int tile, int lane, uint4& hi, uint4& lo) {
  hi = *reinterpret_cast<const uint4*>(buf + tile * TILE + lane * 8);
  lo = *reinterpret_cast<const uint4*>(buf + tile * TILE + 512 + lane * 8);
}

// Stores of one lane's 4 D-layout values (rows r0 + j of a column) with one voffset: the row
// block goes into the descriptor base (rows past the end stay range-checked) and the row j
// into the instruction's immediate offset, so no per-element address registers are kept.
// (Quad-transposing the tile for 16-byte stores measured slower on the serial chain: the DPP
// transposes cost more issue than the store instructions they save.)
__device__ __forceinline__ void st_rows4(bufrsrc r, uint32_t vbase, uint32_t row_bytes, const f32x4& x) {
#pragma unroll
  for (int j = 0; j < 4; ++j) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x[j]), r, vbase + j * row_bytes, 0, 0);
}
// Descriptor over rows [r0, L) of a row-major [rows][D] fp32 block at p (row stride D).
__device__ __forceinline__ bufrsrc rows_from(const float* p, int r0, int L, int D) {
  return make_buf(p + (int64_t)r0 * D, (uint32_t)(L > r0 ? (L - r0) * D * 4 : 0));
}
// The same four values rounded to bf16 (round to nearest even), into a bf16 block.
__device__ __forceinline__ void st_rows4_bf16(bufrsrc r, uint32_t vbase, uint32_t row_bytes, const f32x4& x) {
#pragma unroll
  for (int j = 0; j < 4; ++j) __builtin_amdgcn_raw_buffer_store_b16(f2bf(x[j]), r, vbase + j * row_bytes, 0, 0);
}
__device__ __forceinline__ bufrsrc rows_from_bf16(const void* p, int r0, int L, int D) {
  return make_buf(reinterpret_cast<const bf16_t*>(p) + (int64_t)r0 * D, (uint32_t)(L > r0 ? (L - r0) * D * 2 : 0));
}
// Layout of a per-chunk state copy [K][V] (h, dh; only the chunk backward and the readout read them):
// 16-column blocks, within one the 16-row tiles, within a tile the rows in the order
// (i % 4, (i / 4) % 4), 16 columns each.  A state wave's lane (g4, c16) holds rows 16 ib + 4 g4 + j of
// one column, so each of its 4 stores per tile writes 64 consecutive elements (256 bytes in fp32, 128
// in bf16; in a row-major layout a wave's 16 columns are 64- or 32-byte pieces of 4 rows); 8
// consecutive columns of a row, which the chunk backward loads, stay contiguous.
template <int K>
__device__ __forceinline__ uint32_t hb_off(int i, int v) {
  return ((((uint32_t)(v >> 4) * (K / 16) + (uint32_t)(i >> 4)) * 4 + (uint32_t)(i & 3)) * 4 + (uint32_t)((i >> 2) & 3)) *
             16 + (uint32_t)(v & 15);
}
// A lane's 4 D-layout values (rows 16 ib + 4 g4 + j of column col) of one chunk's [K][V] state block
// at element e0 of p (fp32, or bf16 with B16), in the hb_off layout.
template <int K, int V, bool B16>
__device__ __forceinline__ void st_state4(void* p, int64_t e0, int ib, int g4, int col, const f32x4& x) {
  if constexpr (B16) {
    const bufrsrc r = make_buf(reinterpret_cast<bf16_t*>(p) + e0, K * V * 2);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_amdgcn_raw_buffer_store_b16(f2bf(x[j]), r, hb_off<K>(16 * ib + 4 * g4 + j, col) * 2, 0, 0);
  } else {
    const bufrsrc r = make_buf(reinterpret_cast<float*>(p) + e0, K * V * 4);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x[j]), r, hb_off<K>(16 * ib + 4 * g4 + j, col) * 4, 0, 0);
  }
}
// A lane's 4 D-layout values of 16-row tile `tile` (rows 4 g4 + j of column col) of the row-major
// [rows][D] block whose element e0 is the block's first (fp32, or bf16 with B16; rows past L dropped).
template <bool B16>
__device__ __forceinline__ void st_tile4(void* p, int64_t e0, int tile, int L, int D, int g4, int col,
                                         const f32x4& x) {
  if constexpr (B16)
    st_rows4_bf16(rows_from_bf16(reinterpret_cast<bf16_t*>(p) + e0, 16 * tile, L, D), (4 * g4 * D + col) * 2, D * 2,
                  x);
  else
    st_rows4(rows_from(reinterpret_cast<float*>(p) + e0, 16 * tile, L, D), (4 * g4 * D + col) * 4, D * 4, x);
}

// A sequence of NS fragment-read + MFMA steps with the reads issued LA steps ahead, so the
// LDS latency of step s+LA overlaps the MFMAs of step s.  rd(s, hi, lo) reads step s's A
// fragment; mm(s, hi, lo) issues its MFMAs.  Both are fully unrolled (s is a constant).
template <int NS, int LA, typename Rd, typename Mm>
__device__ __forceinline__ void mfma_pipe(Rd rd, Mm mm) {
  uint4 fh[NS], fl[NS];
#pragma unroll
  for (int s = 0; s < NS + LA; ++s) {
    if (s < NS) rd(s, fh[s], fl[s]);
    if (s >= LA) mm(s - LA, fh[s - LA], fl[s - LA]);
  }
}

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

// ===========================================================================
// Chunk groups (two-level scan).  With NG > 1 groups of m chunks, each state pass runs as
//   pass A  the first group in order (the true state), plus every middle group's affine map
//           S_out = Phi S_in + Psi, taken by running the group from [0 | I] on V + K columns
//           (the Psi columns see U / dO, the Phi columns start at the identity and see none);
//   pass B  state_combine_kernel: the group-start states, serially, S_{g+1} = Phi_g S_g + Psi_g;
//   pass C  every later group from its true incoming state (h / delta stores, final state).
// Pass A's middle groups and pass C's groups all run in parallel, so the serial depth is about
// 2 m + NG chunk steps instead of NT.  The map columns cost K more columns per middle group, so
// the host takes NG > 1 only where B * H leaves CUs idle (kdn_memory.hip, plan_groups).
//   forward:  Sg[g]  = state entering group g (g >= 1);   Mg[g] = [Psi_g | Phi_g] (1 <= g <= NG-2)
//   backward: Sg[g]  = cotangent leaving group g (g <= NG-2), Mg[g] likewise for the reverse map.
// Sg is [BH][NG][K][V], Mg is [BH][NG][K][V + K].
// ===========================================================================
struct GroupPlan {
  int NG;     // number of chunk groups (1: a single serial pass)
  int m;      // chunks per group (the last group may be shorter)
  int pass;   // 0: pass A, 1: pass C (unused when NG == 1)
  float* Sg;
  float* Mg;
  // NG == 1: the pass runs chunks c0 .. c1 - 1 (c1 <= 0: every chunk from c0), entering from h0 (dht)
  // and leaving into ht (dh0); a sequence split into segments runs as consecutive such passes
  int c0 = 0, c1 = 0;
};

// Precision of the per-chunk copies only the backward (and a separate readout) reads, as a bit mask
// (kernel template argument): the forward pass's h (bit 0) and delta (bit 2), the reverse pass's dh
// (bit 1) and d delta (bit 3); a set bit stores the copy in bf16 (rounded once), a clear bit in fp32.
// The recurrences themselves stay fp32 on chip.
enum : int { HB_H = 1, HB_DH = 2, HB_D = 4, HB_DD = 8 };
__device__ __forceinline__ void plan_range(const GroupPlan& P, int g, int NT, int& n0, int& n1) {
  if (P.NG == 1) {
    n0 = P.c0;
    n1 = P.c1 > 0 ? min(P.c1, NT) : NT;
  } else {
    n0 = g * P.m;
    n1 = min(NT, n0 + P.m);
  }
}

// Workgroup -> (bh, column slice, group, role) of a state pass.  `real`: the group is run on the
// true state (stores per-chunk results); otherwise it is a map group.  `phi`: the slice's columns
// are Phi columns (col - V indexes the identity's column).  Returns false for a padding workgroup.
template <int V, int K, bool REVERSE>
__device__ __forceinline__ bool group_task(const GroupPlan& P, int BH, int& bh, int& vs, int& g, bool& real,
                                           bool& phi) {
  constexpr int NV = V / state_cols(V), NS = NV + K / state_cols(V);
  phi = false;
  real = true;
  if (P.NG == 1) {
    xcd_map(blockIdx.x, NV, BH, bh, vs);
    g = 0;
    return true;
  }
  const int G1 = P.NG - 1;
  int u;
  if (P.pass == 0) {
    xcd_map(blockIdx.x, NS, BH * G1, u, vs);
    bh = u / G1;
    const int gi = u % G1;
    if (gi == 0) {  // the group that starts from the true state: first (forward) or last (reverse)
      g = REVERSE ? P.NG - 1 : 0;
      return vs < NV;
    }
    g = gi;
    real = false;
    phi = vs >= NV;
    return true;
  }
  xcd_map(blockIdx.x, NV, BH * G1, u, vs);
  bh = u / G1;
  g = REVERSE ? u % G1 : u % G1 + 1;
  return true;
}

// ===========================================================================
// Forward state pass.  grid: (B*H*V/COLS) for one group, or the pass's task count (GroupPlan);
// block 4 COLS.  LDS 64.5 KB.
// The readout O = Qg h + M delta is left to readout_kernel: it is off the serial chain, and its
// operands (Qg, M) would double the chunk operands staged on the chain's critical path.
// ===========================================================================
// With RO (one chunk group, or pass C of a grouped pass: every workgroup runs a group from its true
// state) the pass also does the readout O = Qg h + M delta of every chunk it runs.
// The block gets four readout waves.  In phase 1 of chunk n each state wave publishes the split B
// fragments of h_n (its state, as it multiplies W with it) and of delta_n to LDS; in phase 2 the
// readout waves multiply them with the A fragments of their 16 chunk rows of Qg and M (loaded from
// HBM one chunk ahead, straight into registers) and store o.  That drops readout_kernel and its
// re-reads of h and delta, and keeps the readout's MFMAs and stores off the serial chain, which only
// pays for the fragment stores.  Both wave groups run the same barrier sequence.
template <int K, int V, typename TO = float, bool RO = false, int HM = 0>
__global__ __launch_bounds__(RO ? 2 * state_threads(V) : state_threads(V), RO ? 1 : 2) void state_fwd_kernel(
    const float* __restrict__ U, const float* __restrict__ W, const float* __restrict__ Kf,
    const float* __restrict__ gc, const float* __restrict__ h0, int T, int H, int NT, int BH,
    float* __restrict__ hbuf, float* __restrict__ Dl, float* __restrict__ ht, GroupPlan P,
    const float* __restrict__ Qg = nullptr, const float* __restrict__ Mg = nullptr, TO* __restrict__ out = nullptr) {
  constexpr int COLS = state_cols(V), NTHR = state_threads(V);
  constexpr int KB = K / 32;           // k-blocks of a contraction over K
  constexpr int ST = K / 16;           // state row tiles per wave
  static_assert((C * K / 4) % NTHR == 0, "staging units per thread");
  constexpr int UN = C * K / 4 / NTHR;  // staging units per thread of a C x K operand
  __shared__ __attribute__((aligned(16))) bf16_t sW[(C / 16) * KB * TILE];        // W: rows c, k = i
  __shared__ __attribute__((aligned(16))) bf16_t sK[(K / 16) * (C / 32) * TILE];  // Kf^T: rows i, k = c
  __shared__ __attribute__((aligned(16))) float sE[K];
  // RO: B fragments of h_n ([wave][kb][hi, lo][lane], K / 32 k-blocks) then of delta_n (2 k-blocks)
  constexpr int NHF = 4 * KB * 2 * 64, NDF = 4 * 2 * 2 * 64;
  __shared__ __attribute__((aligned(16))) uint4 sHD[RO ? NHF + NDF : 1];
  // RO: each readout wave's 16 output rows, regrouped so that every store writes whole row segments
  constexpr int ROWB = COLS * (int)sizeof(TO), QPR = ROWB / 16, RPI = 1024 / ROWB;
  static_assert(ROWB % 128 == 0 && RPI <= 16, "readout rows of 8 or more 16-byte quads");
  __shared__ __attribute__((aligned(16))) uint4 sO[RO ? 4 * 16 * QPR : 1];
  int bh, vs, g;
  bool real, phi;
  if (!group_task<V, K, false>(P, BH, bh, vs, g, real, phi)) return;
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g4 = lane >> 4;
  const int col = vs * COLS + 16 * w + (lane & 15);  // this lane's state column (>= V: a Phi column)
  int n0, n1;
  plan_range(P, g, NT, n0, n1);

  if constexpr (RO) {
    if (tid >= NTHR) {  // readout waves: wave rw owns chunk rows 16 rw .. 16 rw + 15 of all COLS columns
      const int rw = w - 4, r16 = lane & 15;
      const uint32_t c = (uint32_t)(16 * rw + r16);
      float4 rq[KB][2], rm[2][2];
      auto load_QM = [&](int n) {  // this lane's A fragment slots of Qg and M rows (permuted k order)
        const int t0 = n * C, L = min(C, T - t0);
        const bufrsrc rq_ = make_buf(Qg + row_bht(bh, t0, T, K), L * K * 4);  // rows past L read 0
        const bufrsrc rm_ = make_buf(Mg + ((int64_t)bh * NT + n) * C * C, C * C * 4);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) rq[kb][hf] = buf_ld4(rq_, (c * K + 32 * kb + 16 * hf + 4 * g4) * 4);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) rm[kb][hf] = buf_ld4(rm_, (c * C + 32 * kb + 16 * hf + 4 * g4) * 4);
      };
      load_QM(n0);
      __syncthreads();  // the state waves' prologue barrier
      for (int n = n0; n < n1; ++n) {
        const int t0 = n * C, L = min(C, T - t0);
        uint4 qh[KB], ql[KB], mh[2], ml[2];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          const float x[8] = {rq[kb][0].x, rq[kb][0].y, rq[kb][0].z, rq[kb][0].w,
                              rq[kb][1].x, rq[kb][1].y, rq[kb][1].z, rq[kb][1].w};
          split8v(x, qh[kb], ql[kb]);
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const float x[8] = {rm[kb][0].x, rm[kb][0].y, rm[kb][0].z, rm[kb][0].w,
                              rm[kb][1].x, rm[kb][1].y, rm[kb][1].z, rm[kb][1].w};
          split8v(x, mh[kb], ml[kb]);
        }
        if (n + 1 < n1) load_QM(n + 1);
        __syncthreads();  // end of phase 1: h_n and delta_n fragments published
        const bufrsrc ro = make_buf(out + row_bthk(b, t0, h, T, H, V), (uint32_t)((L - 1) * H + 1) * V * sizeof(TO));
        const int qr = lane & 3;
        // this wave's rows; the barriers of each chunk separate the last chunk's reads from these writes
        unsigned char* sOw = reinterpret_cast<unsigned char*>(sO) + rw * 16 * ROWB;
#pragma unroll
        for (int sw = 0; sw < 4; ++sw) {  // the 16 columns of state wave sw (four independent chains)
          f32x4 O = zero4();
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) {
            const uint4 bh2 = sHD[((sw * KB + kb) * 2) * 64 + lane], bl2 = sHD[((sw * KB + kb) * 2 + 1) * 64 + lane];
            O = mma3(qh[kb], ql[kb], bh2, bl2, O);
          }
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) {
            if (kb == 1 && rw < 2) continue;  // M[c][s] = 0 for s > c
            const uint4 dh2 = sHD[NHF + ((sw * 2 + kb) * 2) * 64 + lane], dl2 = sHD[NHF + ((sw * 2 + kb) * 2 + 1) * 64 + lane];
            O = mma3(mh[kb], ml[kb], dh2, dl2, O);
          }
          // lane (column 4 q + r, rows 4 g4 ..) -> quad transpose -> row 4 g4 + r, columns 4 q .. 4 q + 3,
          // into this wave's LDS rows (16-byte quad j of row r at slot j ^ (r & 7))
          const float4 y = quad_transpose(float4{O[0], O[1], O[2], O[3]}, qr);
          const int r = 4 * g4 + qr, cb = (16 * sw + 4 * ((lane & 15) >> 2)) * (int)sizeof(TO);
          unsigned char* dst = sOw + r * ROWB + (((cb >> 4) ^ (r & 7)) << 4) + (cb & 15);
          if constexpr (sizeof(TO) == 2) {
            *reinterpret_cast<u32x2*>(dst) =
                u32x2{(uint32_t)f2bf(y.x) | ((uint32_t)f2bf(y.y) << 16), (uint32_t)f2bf(y.z) | ((uint32_t)f2bf(y.w) << 16)};
          } else {
            *reinterpret_cast<float4*>(dst) = y;
          }
        }
        wave_lds_sync();
#pragma unroll
        for (int hh = 0; hh < 16 / RPI; ++hh) {  // RPI whole rows of COLS columns per store
          const int rr = lane / QPR + RPI * hh, qd = lane % QPR;
          const u32x4 x = *reinterpret_cast<const u32x4*>(sOw + rr * ROWB + ((qd ^ (rr & 7)) << 4));
          const uint32_t eb =
              ((uint32_t)((16 * rw + rr) * H) * V + (uint32_t)(vs * COLS)) * (uint32_t)sizeof(TO) + 16 * qd;
          __builtin_amdgcn_raw_buffer_store_b128(x, ro, eb, 0, 0);  // rows past L dropped
        }
        __syncthreads();  // end of phase 2: the fragments may be overwritten
      }
      return;
    }
  }

  float4 rW[UN];
  float rK[UN][4], rU[4][4], rE = 0.f;
  auto load_W = [&](int n) {  // W (rows c, k = i)
    const int t0 = n * C, L = min(C, T - t0);
    const bufrsrc rw = make_buf(W + row_bht(bh, t0, T, K), L * K * 4);  // rows past L read 0
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const Unit x = unit<K>(tid + NTHR * u);
      rW[u] = buf_ld4(rw, (x.row * K + x.k0) * 4);
    }
  };
  auto load_K = [&](int n) {  // Kf^T (rows i, k = c), U rows of this lane, e^{g_last}
    const int t0 = n * C, L = min(C, T - t0);
    const bufrsrc rk = make_buf(Kf + row_bht(bh, t0, T, K), L * K * 4);
    const bufrsrc ru = make_buf(U + row_bht(bh, t0, T, V), phi ? 0u : L * V * 4);  // Phi columns: U = 0
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const Unit x = unit<C>(tid + NTHR * u);
#pragma unroll
      for (int j = 0; j < 4; ++j) rK[u][j] = buf_ld(rk, ((x.k0 + j) * K + x.row) * 4);
    }
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
      for (int j = 0; j < 4; ++j) rU[cb][j] = buf_ld(ru, ((16 * cb + 4 * g4 + j) * V + col) * 4);
    {  // raw g_last of the chunk; the exponential is taken when staging, so no wait sits here
      const bufrsrc rg = make_buf(gc + row_bthk(b, t0 + L - 1, h, T, H, K), K * 4);  // lanes >= K read 0
      rE = buf_ld(rg, tid * 4);
    }
  };
  auto stage_W = [&]() {
#pragma unroll
    for (int u = 0; u < UN; ++u) put_unit(sW, unit<K>(tid + NTHR * u).off, rW[u].x, rW[u].y, rW[u].z, rW[u].w);
  };
  auto stage_K = [&]() {
#pragma unroll
    for (int u = 0; u < UN; ++u) put_unit(sK, unit<C>(tid + NTHR * u).off, rK[u][0], rK[u][1], rK[u][2], rK[u][3]);
    if (tid < K) sE[tid] = fexp2(rE);
  };

  // the state entering the group: h0 (or 0) for the first group, the combined group-start state for
  // a later group, [0 | I] for a map group
  f32x4 S[ST];
  {
    const float* src = !real ? nullptr
                       : g == 0 ? (h0 ? h0 + (int64_t)bh * K * V : nullptr)
                                : P.Sg + ((int64_t)bh * P.NG + g) * K * V;
#pragma unroll
    for (int ib = 0; ib < ST; ++ib)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = 16 * ib + 4 * g4 + j;
        S[ib][j] = src ? src[(int64_t)row * V + col] : (phi && row == col - V ? 1.f : 0.f);
      }
  }

  load_W(n0);
  stage_W();
  load_K(n0);
  __syncthreads();
  for (int n = n0; n < n1; ++n) {
    const int t0 = n * C, L = min(C, T - t0);
    if (real && hbuf) {  // (no h, delta stores when the readout is fused and no backward follows)
      const int64_t e0 = ((int64_t)bh * NT + n) * K * V;
#pragma unroll
      for (int ib = 0; ib < ST; ++ib) st_state4<K, V, (HM & HB_H) != 0>(hbuf, e0, ib, g4, col, S[ib]);
    }

    // ---- phase 1: delta = U - W S   (reads sW; fills sK with chunk n; loads W of chunk n+1)
    stage_K();
    float cU[4][4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
      for (int j = 0; j < 4; ++j) cU[cb][j] = rU[cb][j];
    if (n + 1 < n1) load_W(n + 1);
    f32x4 D[4];
    {
      uint4 bh_[KB], bl_[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) bfrag(S[2 * kb], S[2 * kb + 1], bh_[kb], bl_[kb]);
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) D[cb] = zero4();
      // step s: kb = s / 4, cb = s % 4
      mfma_pipe<4 * KB, 2>([&](int st, uint4& ah, uint4& al) { afrag(sW, (st & 3) * KB + (st >> 2), lane, ah, al); },
                           [&](int st, const uint4& ah, const uint4& al) {
                             D[st & 3] = mma3(ah, al, bh_[st >> 2], bl_[st >> 2], D[st & 3]);
                           });
#pragma unroll
      for (int cb = 0; cb < 4; ++cb)
#pragma unroll
        for (int j = 0; j < 4; ++j) D[cb][j] = cU[cb][j] - D[cb][j];
      if (real && Dl) {
        const int64_t e0 = row_bht(bh, t0, T, V);
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
          st_tile4<(HM & HB_D) != 0>(Dl, e0, cb, L, V, g4, col, D[cb]);  // rows past L dropped
      }
      if constexpr (RO) {  // publish the B fragments of h_n (multiplied with W above) and delta_n
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          sHD[((w * KB + kb) * 2) * 64 + lane] = bh_[kb];
          sHD[((w * KB + kb) * 2 + 1) * 64 + lane] = bl_[kb];
        }
        uint4 dh2, dl2;
        bfrag(D[0], D[1], dh2, dl2);
        sHD[NHF + ((w * 2) * 2) * 64 + lane] = dh2;
        sHD[NHF + ((w * 2) * 2 + 1) * 64 + lane] = dl2;
        bfrag(D[2], D[3], dh2, dl2);
        sHD[NHF + ((w * 2 + 1) * 2) * 64 + lane] = dh2;
        sHD[NHF + ((w * 2 + 1) * 2 + 1) * 64 + lane] = dl2;
      }
    }
    __syncthreads();

    // ---- phase 2: S = e S + Kf^T delta   (reads sK; fills sW with chunk n+1; loads Kf, U, e of n+1)
    if (n + 1 < n1) {
      stage_W();
      load_K(n + 1);
    }
    {
      uint4 dh_[2], dl_[2];
      bfrag(D[0], D[1], dh_[0], dl_[0]);
      bfrag(D[2], D[3], dh_[1], dl_[1]);
#pragma unroll
      for (int ib = 0; ib < ST; ++ib) {
        const float4 e = *reinterpret_cast<const float4*>(sE + 16 * ib + 4 * g4);
        S[ib] = f32x4{e.x * S[ib][0], e.y * S[ib][1], e.z * S[ib][2], e.w * S[ib][3]};
      }
      // step s: S[ib] += Kf^T delta (kb = s / ST, ib = s % ST)
      mfma_pipe<2 * ST, 2>([&](int st, uint4& ah, uint4& al) { afrag(sK, (st % ST) * 2 + st / ST, lane, ah, al); },
                           [&](int st, const uint4& ah, const uint4& al) {
                             S[st % ST] = mma3(ah, al, dh_[st / ST], dl_[st / ST], S[st % ST]);
                           });
    }
    __syncthreads();
  }
  // the state leaving the group: the final state (last group), the next group's start (first group
  // of a grouped pass), or the group map [Psi | Phi]
  float* dst = nullptr;
  int64_t ld = V;
  if (!real) {
    dst = P.Mg + ((int64_t)bh * P.NG + g) * K * (V + K);
    ld = V + K;
  } else if (g == P.NG - 1) {
    dst = ht ? ht + (int64_t)bh * K * V : nullptr;
  } else if (g == 0) {
    dst = P.Sg + ((int64_t)bh * P.NG + 1) * K * V;
  }
  if (dst) {
#pragma unroll
    for (int ib = 0; ib < ST; ++ib)
#pragma unroll
      for (int j = 0; j < 4; ++j) dst[(int64_t)(16 * ib + 4 * g4 + j) * ld + col] = S[ib][j];
  }
}

// ===========================================================================
// Forward readout, chunk-parallel:  O = Qg h + M delta  per chunk, from the state pass's h (the
// state entering the chunk) and delta, for the first NR chunks of every head (NR = NT: all of them;
// a grouped pass whose later groups read out in pass C: the first group's).  grid: one workgroup per
// (chunk, head, 64 columns of V), see below; block 256, LDS 48 KB.
// Computed transposed, O^T = h^T Qg^T + delta^T M^T, so each lane's D tile holds 4 consecutive
// columns of one chunk row (8- or 16-byte stores).  h^T and delta^T (A operands, contraction over
// the state row i / the chunk row s) are staged once per workgroup as split fragments in LDS; the
// B operands Qg^T and M^T are rows of Qg and M, loaded straight into registers by the wave that
// owns those 16 chunk rows.  Fragment k order is natural (slot j of lane group g <-> k = 8 g + j).
// ===========================================================================
template <int K, int V, typename TO, int HM = 0>
__global__ __launch_bounds__(256, 3) void readout_kernel(const float* __restrict__ Qg, const float* __restrict__ Mg,
                                                         const float* __restrict__ hbuf, const float* __restrict__ Dl,
                                                         int T, int H, int NT, int NR, int BH, TO* __restrict__ out) {
  constexpr int VC = 64;                 // columns of V per workgroup
  constexpr int KB = K / 32, VT = VC / 16;
  static_assert(V % VC == 0, "V is a multiple of 64");
  __shared__ __attribute__((aligned(16))) bf16_t sH[VT * KB * TILE];  // h^T: rows v, k = i
  __shared__ __attribute__((aligned(16))) bf16_t sD[VT * 2 * TILE];   // delta^T: rows v, k = s
  // workgroup lin -> (chunk of a head, V half): the two halves of a chunk are lin and lin + 8, which
  // dispatch round-robin puts on one XCD, so they share Qg and M through its L2
  static_assert(V / VC == 2 || V / VC == 1, "one or two column halves");
  const int lin = blockIdx.x, NH = V / VC;
  const int ch = NH == 2 ? 8 * (lin >> 4) + (lin & 7) : lin, half = NH == 2 ? (lin >> 3) & 1 : 0;
  if (ch >= NR * BH) return;  // the first NR chunks of each head (NR = NT: all)
  const int n = ch % NR, bh = ch / NR, v0 = VC * half, b = bh / H, h = bh % H;
  const int t0 = n * C, L = min(C, T - t0);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r16 = lane & 15, g4 = lane >> 4;
  const int64_t chunk = (int64_t)bh * NT + n;

  // ---- B operands of this wave's 16 chunk rows c = 16 w + r16: Qg row (k = i) and M row (k = s)
  const uint32_t c = (uint32_t)(16 * w + r16);
  const bufrsrc rQ = make_buf(Qg + ((int64_t)bh * T + t0) * K, L * K * 4);
  const bufrsrc rM = make_buf(Mg + chunk * C * C, C * C * 4);
  float4 q4[KB][2], m4[2][2];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb)
#pragma unroll
    for (int p = 0; p < 2; ++p) q4[kb][p] = buf_ld4(rQ, (c * K + 32 * kb + 8 * g4 + 4 * p) * 4);
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int p = 0; p < 2; ++p) m4[kb][p] = buf_ld4(rM, (c * C + 32 * kb + 8 * g4 + 4 * p) * 4);

  // ---- stage h^T and delta^T.  A wave loads 4 rows x 64 columns per instruction (lane l: row
  // 4 rb + l % 4, columns 4 (l / 4) .. +3), transposes each 4 x 4 block across its lane quad (DPP),
  // so a lane holds 4 consecutive rows of one column: 4 consecutive fragment slots of one lane,
  // written as 8 bytes of hi and 8 of lo
  {
    constexpr int EH = (HM & HB_H) ? 2 : 4, ED = (HM & HB_D) ? 2 : 4;  // bytes per stored element
    const bufrsrc rh = make_buf(reinterpret_cast<const char*>(hbuf) + chunk * K * V * EH, K * V * EH);
    const bufrsrc rd = make_buf(reinterpret_cast<const char*>(Dl) + ((int64_t)bh * T + t0) * V * ED,
                                L * V * ED);  // rows past L read 0
    constexpr int HU = K / 16, DU = C / 16;  // 4-row blocks per wave
    const int qr = lane & 3, vq = 4 * (lane >> 2), vc = vq + qr;  // after the transpose: column vc
    float4 hx[HU], dx[DU];
    auto ld4h = [&](bufrsrc r, uint32_t e, auto b16) {  // 4 consecutive elements of either precision
      if constexpr (!decltype(b16)::value) {
        return buf_ld4(r, e * 4);
      } else {
        const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, e * 2, 0, 0);
        return float4{__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u), __uint_as_float(v.y << 16),
                      __uint_as_float(v.y & 0xffff0000u)};
      }
    };
#pragma unroll
    for (int u = 0; u < HU; ++u) {
      const int hi = 4 * (w + 4 * u) + qr, hv = v0 + vq;
      hx[u] = ld4h(rh, hb_off<K>(hi, hv), std::integral_constant<bool, (HM & HB_H) != 0>{});
    }
#pragma unroll
    for (int u = 0; u < DU; ++u)
      dx[u] = ld4h(rd, (4 * (w + 4 * u) + qr) * V + v0 + vq, std::integral_constant<bool, (HM & HB_D) != 0>{});
    auto put = [&](bf16_t* buf, int nkb, int r0, const float4& x) {  // rows r0 .. r0+3 of column vc
      const float4 y = quad_transpose(x, qr);
      const int tile = (vc >> 4) * nkb + (r0 >> 5), ln = (vc & 15) + 16 * ((r0 & 31) >> 3);
      uint32_t h0, l0, h1, l1;
      split2(y.x, y.y, h0, l0);
      split2(y.z, y.w, h1, l1);
      const int off = tile * TILE + ln * 8 + (r0 & 7);
      *reinterpret_cast<uint2*>(buf + off) = uint2{h0, h1};
      *reinterpret_cast<uint2*>(buf + off + 512) = uint2{l0, l1};
    };
#pragma unroll
    for (int u = 0; u < HU; ++u) put(sH, KB, 4 * (w + 4 * u), hx[u]);
#pragma unroll
    for (int u = 0; u < DU; ++u) put(sD, 2, 4 * (w + 4 * u), dx[u]);
  }
  uint4 qh[KB], ql[KB], mh[2], ml[2];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const float x[8] = {q4[kb][0].x, q4[kb][0].y, q4[kb][0].z, q4[kb][0].w,
                        q4[kb][1].x, q4[kb][1].y, q4[kb][1].z, q4[kb][1].w};
    split8v(x, qh[kb], ql[kb]);
  }
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const float x[8] = {m4[kb][0].x, m4[kb][0].y, m4[kb][0].z, m4[kb][0].w,
                        m4[kb][1].x, m4[kb][1].y, m4[kb][1].z, m4[kb][1].w};
    split8v(x, mh[kb], ml[kb]);
  }
  __syncthreads();

  // ---- O^T tiles (v tile vt, chunk rows 16 w ..): M[c][s] = 0 for s > c, so chunk-row tiles 0, 1
  // skip the second s block
  const int r0 = 16 * w;
  const bufrsrc ro = make_buf(out + row_bthk(b, t0 + r0, h, T, H, V),
                              L > r0 ? ((L - 1 - r0) * H + 1) * V * (uint32_t)sizeof(TO) : 0u);
#pragma unroll
  for (int vt = 0; vt < VT; ++vt) {
    f32x4 acc = zero4();
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      uint4 ah, al;
      afrag(sH, vt * KB + kb, lane, ah, al);
      acc = mma3(ah, al, qh[kb], ql[kb], acc);
    }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      if (kb == 1 && w < 2) continue;
      uint4 ah, al;
      afrag(sD, vt * 2 + kb, lane, ah, al);
      acc = mma3(ah, al, mh[kb], ml[kb], acc);
    }
    const uint32_t e = (uint32_t)(r16 * H) * V + v0 + 16 * vt + 4 * g4;  // rows past L dropped
    if constexpr (sizeof(TO) == 2) {
      __builtin_amdgcn_raw_buffer_store_b64(
          u32x2{(uint32_t)f2bf(acc[0]) | ((uint32_t)f2bf(acc[1]) << 16), (uint32_t)f2bf(acc[2]) | ((uint32_t)f2bf(acc[3]) << 16)},
          ro, e * 2, 0, 0);
    } else {
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc), ro, e * 4, 0, 0);
    }
  }
}

// ===========================================================================
// Reverse state pass.  grid: (B*H*V/COLS) for one group, or the pass's task count (GroupPlan);
// block 4 COLS.  LDS 112.5 KB.
// With HW the block gets four helper waves (block 8 COLS, LDS 128.5 KB).  The products M^T dO and
// Qg^T dO do not depend on the recurrence, so the helpers compute them one phase ahead of the state
// waves and hand them over through LDS in the state waves' D layout: Qg^T dO of chunk n during
// phase 1 of chunk n (added to dS in phase 2), M^T dO of chunk n - 1 during phase 2 of chunk n
// (added to d delta in phase 1 of chunk n - 1).  Helper wave hw owns the row tiles of those
// products (Qg^T row tiles hw ST/4 .., M^T row tile hw) for all four column groups: their A
// fragments (columns of Qg and M) are loaded straight into registers, one chunk ahead; each helper
// loads dO of one column group and publishes its B fragments to the others through LDS.  The state
// waves then stage only Kf and W^T and issue 32 split products per chunk instead of 56.  Both wave
// groups run the same barrier sequence: two in the prologue, two per chunk.
// ===========================================================================
template <int K, int V, typename TDO, bool HW = false, int HM = 0>
__global__ __launch_bounds__(HW ? 2 * state_threads(V) : state_threads(V)) void state_bwd_kernel(
    const float* __restrict__ Mg, const float* __restrict__ Kf, const float* __restrict__ Qg,
    const float* __restrict__ W, const float* __restrict__ gc, const TDO* __restrict__ dO,
    const float* __restrict__ dht, int T, int H, int NT, int BH, float* __restrict__ dhbuf,
    float* __restrict__ dDl, float* __restrict__ dh0, GroupPlan P) {
  constexpr int COLS = state_cols(V), NTHR = state_threads(V);
  constexpr int KB = K / 32;
  constexpr int ST = K / 16;
  static_assert((C * K / 4) % NTHR == 0 && (C * C / 4) % NTHR == 0, "staging units per thread");
  static_assert(!HW || (COLS == 64 && ST % 4 == 0), "helper waves: four state waves, K a multiple of 64");
  constexpr int UN = C * K / 4 / NTHR;  // staging units per thread of a C x K operand
  constexpr int UM = C * C / 4 / NTHR;  // ... of M^T
  constexpr bool DO_BF16 = sizeof(TDO) == 2;
  // phase 1: M^T (rows c', k = c) and Kf (rows c, k = i);  phase 2: Qg^T, W^T (rows i, k = c).
  // HW: M^T and Qg^T are not staged; the helpers' products and dO fragments take their place.
  __shared__ __attribute__((aligned(16))) bf16_t sM[HW ? 8 : (C / 16) * (C / 32) * TILE];
  __shared__ __attribute__((aligned(16))) bf16_t sKn[(C / 16) * KB * TILE];
  __shared__ __attribute__((aligned(16))) bf16_t sQ[HW ? 8 : (K / 16) * (C / 32) * TILE];
  __shared__ __attribute__((aligned(16))) bf16_t sWt[(K / 16) * (C / 32) * TILE];
  __shared__ __attribute__((aligned(16))) float sE[K];
  __shared__ f32x4 sPA[HW ? 4 * 4 * 64 : 1];   // M^T dO: [state wave][row tile cb][lane]
  __shared__ f32x4 sPB[HW ? 4 * ST * 64 : 1];  // Qg^T dO: [state wave][row tile ib][lane]
  __shared__ uint4 sO[HW ? 4 * 2 * 2 * 64 : 1];  // dO B fragments: [column group][kb][hi, lo][lane]
  int bh, vs, g;
  bool real, phi;
  if (!group_task<V, K, true>(P, BH, bh, vs, g, real, phi)) return;
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g4 = lane >> 4;
  int n0, n1;
  plan_range(P, g, NT, n0, n1);

  // dO as loaded (raw bf16 bits or fp32), widened only where the fragments are built, so the
  // loads of a chunk are all issued before any of them is waited for
  using RawO = std::conditional_t<DO_BF16, uint16_t, float>;
  auto widen = [](RawO x) -> float {
    if constexpr (DO_BF16) return bf2f(x);
    else return x;
  };
  // dO rows 4 g4 + j (+ 16 cb) of column `col` of chunk n (rows past L and Phi columns read 0)
  auto load_dO = [&](int n, int col, RawO (&rO)[4][4]) {
    const int t0 = n * C, L = min(C, T - t0);
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      // dO rows 16 cb .. are H*V apart; the descriptor ends right after row L-1's head h
      const int r0 = 16 * cb;
      const bufrsrc ro = make_buf(dO + row_bthk(b, t0 + r0, h, T, H, V),
                                  (!phi && L > r0) ? ((L - 1 - r0) * H + 1) * V * (uint32_t)sizeof(TDO) : 0u);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t e = (uint32_t)((4 * g4 + j) * H * V + col);
        if constexpr (DO_BF16) rO[cb][j] = __builtin_amdgcn_raw_buffer_load_b16(ro, e * 2, 0, 0);
        else rO[cb][j] = buf_ld(ro, e * 4);
      }
    }
  };
  // the B fragments (k = c) of those rows; a bf16 dO has ol = 0
  auto dO_frags = [&](const RawO (&rO)[4][4], uint4 (&oh)[2], uint4 (&ol)[2]) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
      bfrag(f32x4{widen(rO[2 * kb][0]), widen(rO[2 * kb][1]), widen(rO[2 * kb][2]), widen(rO[2 * kb][3])},
            f32x4{widen(rO[2 * kb + 1][0]), widen(rO[2 * kb + 1][1]), widen(rO[2 * kb + 1][2]),
                  widen(rO[2 * kb + 1][3])},
            oh[kb], ol[kb]);
  };

  if constexpr (HW) {
    if (tid >= NTHR) {
      constexpr int RT = ST / 4;  // Qg^T row tiles per helper wave
      const int hw = w - 4, r16 = lane & 15;
      // A fragment slot s of lane group g4 in k-block kb: chunk row c = 32 kb + 4 g4 + s (s < 4) or
      // 32 kb + 16 + 4 g4 + s - 4
      auto crow = [&](int kb, int s) { return (uint32_t)(32 * kb + 16 * (s >> 2) + 4 * g4 + (s & 3)); };
      float rq[RT][2][8], rm[2][8];
      RawO rO[4][4];
      auto load_Q = [&](int n) {  // Qg^T rows i = 16 (hw RT + t) + r16: Qg[c][i]
        const int t0 = n * C, L = min(C, T - t0);
        const bufrsrc r = make_buf(Qg + row_bht(bh, t0, T, K), L * K * 4);  // rows past L read 0
#pragma unroll
        for (int t = 0; t < RT; ++t)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int s = 0; s < 8; ++s)
              rq[t][kb][s] = buf_ld(r, (crow(kb, s) * K + (uint32_t)(16 * (hw * RT + t) + r16)) * 4);
      };
      auto load_M = [&](int n) {  // M^T rows c' = 16 hw + r16: M[c][c'] (k-block 0 is zero for hw >= 2)
        const bufrsrc r = make_buf(Mg + ((int64_t)bh * NT + n) * C * C, C * C * 4);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int s = 0; s < 8; ++s)
            rm[kb][s] = (kb == 0 && hw >= 2) ? 0.f : buf_ld(r, (crow(kb, s) * C + (uint32_t)(16 * hw + r16)) * 4);
      };
      const int ocol = vs * COLS + 16 * hw + r16;  // the column group whose dO this wave loads
      auto publish_O = [&]() {
        uint4 oh[2], ol[2];
        dO_frags(rO, oh, ol);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          sO[((hw * 2 + kb) * 2) * 64 + lane] = oh[kb];
          if constexpr (!DO_BF16) sO[((hw * 2 + kb) * 2 + 1) * 64 + lane] = ol[kb];
        }
      };
      uint4 foh[4][2], fol[4][2];  // dO fragments of all four column groups
      auto read_O = [&]() {
#pragma unroll
        for (int sw = 0; sw < 4; ++sw)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) {
            foh[sw][kb] = sO[((sw * 2 + kb) * 2) * 64 + lane];
            if constexpr (!DO_BF16) fol[sw][kb] = sO[((sw * 2 + kb) * 2 + 1) * 64 + lane];
          }
      };
      auto prod = [&](const uint4& ah, const uint4& al, int sw, int kb, f32x4 acc) {
        if constexpr (DO_BF16) return mma2(ah, al, foh[sw][kb], acc);
        else return mma3(ah, al, foh[sw][kb], fol[sw][kb], acc);
      };
      auto product_A = [&]() {  // M^T dO (row tile hw) -> sPA
        uint4 mh[2], ml[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) split8v(rm[kb], mh[kb], ml[kb]);
#pragma unroll
        for (int sw = 0; sw < 4; ++sw) {
          f32x4 acc = zero4();
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) {
            if (kb == 0 && hw >= 2) continue;  // M^T[c'][c] = 0 for c < c'
            acc = prod(mh[kb], ml[kb], sw, kb, acc);
          }
          sPA[(sw * 4 + hw) * 64 + lane] = acc;
        }
      };
      auto product_B = [&]() {  // Qg^T dO (row tiles hw RT ..) -> sPB
#pragma unroll
        for (int t = 0; t < RT; ++t) {
          uint4 qh[2], ql[2];
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) split8v(rq[t][kb], qh[kb], ql[kb]);
#pragma unroll
          for (int sw = 0; sw < 4; ++sw) {
            f32x4 acc = zero4();
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) acc = prod(qh[kb], ql[kb], sw, kb, acc);
            sPB[(sw * ST + hw * RT + t) * 64 + lane] = acc;
          }
        }
      };
      const int nl = n1 - 1;
      load_dO(nl, ocol, rO);
      load_M(nl);
      load_Q(nl);
      publish_O();
      __syncthreads();  // prologue 1: dO fragments of chunk nl
      read_O();
      product_A();
      if (nl > n0) {
        load_dO(nl - 1, ocol, rO);
        load_M(nl - 1);
      }
      __syncthreads();  // prologue 2: M^T dO of chunk nl
      for (int n = nl; n >= n0; --n) {
        // phase 1: Qg^T dO of chunk n; dO fragments of chunk n - 1
        product_B();
        if (n > n0) {
          load_Q(n - 1);
          publish_O();
        }
        __syncthreads();
        // phase 2: M^T dO of chunk n - 1
        if (n > n0) {
          read_O();
          product_A();
          if (n - 1 > n0) {
            load_dO(n - 2, ocol, rO);
            load_M(n - 2);
          }
        }
        __syncthreads();
      }
      return;
    }
  }

  const int col = vs * COLS + 16 * w + (lane & 15);  // >= V: a Phi column (its dO is zero)
  float rM[HW ? 1 : UM][4], rQ[HW ? 1 : UN][4], rWt[UN][4], rE = 0.f;
  RawO rO[4][4];
  float4 rKn[UN];
  auto load_p1 = [&](int n) {  // M^T and Kf of chunk n
    const int t0 = n * C, L = min(C, T - t0);
    if constexpr (!HW) {
      const bufrsrc rm = make_buf(Mg + ((int64_t)bh * NT + n) * C * C, C * C * 4);  // M[c][c'] row-major
#pragma unroll
      for (int u = 0; u < UM; ++u) {
        const Unit x = unit<C>(tid + NTHR * u);  // row = c' (the d delta index), k = c
#pragma unroll
        for (int j = 0; j < 4; ++j) rM[u][j] = buf_ld(rm, ((x.k0 + j) * C + x.row) * 4);
      }
    }
    const bufrsrc rk = make_buf(Kf + row_bht(bh, t0, T, K), L * K * 4);
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const Unit x = unit<K>(tid + NTHR * u);
      rKn[u] = buf_ld4(rk, (x.row * K + x.k0) * 4);
    }
  };
  auto load_p2 = [&](int n) {  // Qg^T, W^T, dO rows of this lane, e^{g_last} of chunk n
    const int t0 = n * C, L = min(C, T - t0);
    const bufrsrc rq = make_buf(Qg + row_bht(bh, t0, T, K), L * K * 4);
    const bufrsrc rw = make_buf(W + row_bht(bh, t0, T, K), L * K * 4);
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const Unit x = unit<C>(tid + NTHR * u);  // row = i, k = c
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t o = ((x.k0 + j) * K + x.row) * 4;
        if constexpr (!HW) rQ[u][j] = buf_ld(rq, o);
        rWt[u][j] = buf_ld(rw, o);
      }
    }
    if constexpr (!HW) load_dO(n, col, rO);
    {  // raw g_last of the chunk; the exponential is taken when staging, so no wait sits here
      const bufrsrc rg = make_buf(gc + row_bthk(b, t0 + L - 1, h, T, H, K), K * 4);  // lanes >= K read 0
      rE = buf_ld(rg, tid * 4);
    }
  };
  auto stage_p1 = [&]() {
    if constexpr (!HW) {
#pragma unroll
      for (int u = 0; u < UM; ++u) put_unit(sM, unit<C>(tid + NTHR * u).off, rM[u][0], rM[u][1], rM[u][2], rM[u][3]);
    }
#pragma unroll
    for (int u = 0; u < UN; ++u)
      put_unit(sKn, unit<K>(tid + NTHR * u).off, rKn[u].x, rKn[u].y, rKn[u].z, rKn[u].w);
  };
  auto stage_p2 = [&]() {
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const int off = unit<C>(tid + NTHR * u).off;
      if constexpr (!HW) put_unit(sQ, off, rQ[u][0], rQ[u][1], rQ[u][2], rQ[u][3]);
      put_unit(sWt, off, rWt[u][0], rWt[u][1], rWt[u][2], rWt[u][3]);
    }
    if (tid < K) sE[tid] = fexp2(rE);
  };

  // the cotangent leaving the group: dht (or 0) for the last group, the combined one for an earlier
  // group, [0 | I] for a map group
  f32x4 dS[ST];
  {
    const float* src = !real ? nullptr
                       : g == P.NG - 1 ? (dht ? dht + (int64_t)bh * K * V : nullptr)
                                       : P.Sg + ((int64_t)bh * P.NG + g) * K * V;
#pragma unroll
    for (int ib = 0; ib < ST; ++ib)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = 16 * ib + 4 * g4 + j;
        dS[ib][j] = src ? src[(int64_t)row * V + col] : (phi && row == col - V ? 1.f : 0.f);
      }
  }

  load_p1(n1 - 1);
  stage_p1();
  load_p2(n1 - 1);
  if constexpr (HW) __syncthreads();  // the helpers' first barrier
  __syncthreads();
  for (int n = n1 - 1; n >= n0; --n) {
    const int t0 = n * C, L = min(C, T - t0);
    if (real) {
      const int64_t e0 = ((int64_t)bh * NT + n) * K * V;
#pragma unroll
      for (int ib = 0; ib < ST; ++ib) st_state4<K, V, (HM & HB_DH) != 0>(dhbuf, e0, ib, g4, col, dS[ib]);
    }

    // dO of this chunk as B fragments (k = c), kept for both phases
    uint4 oh[2], ol[2];
    if constexpr (!HW) dO_frags(rO, oh, ol);

    // ---- phase 1: d delta = M^T dO + Kf dS   (reads sM, sKn; fills sQ, sWt with chunk n)
    stage_p2();
    if (n > n0) load_p1(n - 1);
    f32x4 dD[4];
    {
      uint4 bh_[KB], bl_[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) bfrag(dS[2 * kb], dS[2 * kb + 1], bh_[kb], bl_[kb]);
      if constexpr (HW) {
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) dD[cb] = sPA[(w * 4 + cb) * 64 + lane];
        // step m: Kf dS (kb = m / 4, cb = m % 4)
        mfma_pipe<4 * KB, 2>([&](int st, uint4& ah, uint4& al) { afrag(sKn, (st & 3) * KB + (st >> 2), lane, ah, al); },
                             [&](int st, const uint4& ah, const uint4& al) {
                               dD[st & 3] = mma3(ah, al, bh_[st >> 2], bl_[st >> 2], dD[st & 3]);
                             });
      } else {
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) dD[cb] = zero4();
        // steps 0..5: M^T dO over the nonzero tiles (cb, kb): (0,0) (1,0) (0,1) (1,1) (2,1) (3,1)
        // (M^T[c'][c] = M[c][c'] = 0 for c < c'); then Kf dS (kb = m / 4, cb = m % 4)
        mfma_pipe<6 + 4 * KB, 2>(
            [&](int st, uint4& ah, uint4& al) {
              if (st < 6) {
                const int cb = st < 2 ? st : st - 2, kb = st < 2 ? 0 : 1;
                afrag(sM, cb * 2 + kb, lane, ah, al);
              } else {
                const int m = st - 6;
                afrag(sKn, (m & 3) * KB + (m >> 2), lane, ah, al);
              }
            },
            [&](int st, const uint4& ah, const uint4& al) {
              if (st < 6) {
                const int cb = st < 2 ? st : st - 2, kb = st < 2 ? 0 : 1;
                dD[cb] = DO_BF16 ? mma2(ah, al, oh[kb], dD[cb]) : mma3(ah, al, oh[kb], ol[kb], dD[cb]);
              } else {
                const int m = st - 6, cb = m & 3, kb = m >> 2;
                dD[cb] = mma3(ah, al, bh_[kb], bl_[kb], dD[cb]);
              }
            });
      }
      if (real) {
        const int64_t e0 = row_bht(bh, t0, T, V);
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
          st_tile4<(HM & HB_DD) != 0>(dDl, e0, cb, L, V, g4, col, dD[cb]);  // rows past L dropped
      }
    }
    __syncthreads();

    // ---- phase 2: dS <- e dS + Qg^T dO - W^T d delta   (reads sQ, sWt; fills sM, sKn with n-1)
    if (n > n0) {
      stage_p1();
      load_p2(n - 1);
    }
    {
      uint4 dh_[2], dl_[2];
      bfrag(-dD[0], -dD[1], dh_[0], dl_[0]);
      bfrag(-dD[2], -dD[3], dh_[1], dl_[1]);
#pragma unroll
      for (int ib = 0; ib < ST; ++ib) {
        const float4 e = *reinterpret_cast<const float4*>(sE + 16 * ib + 4 * g4);
        dS[ib] = f32x4{e.x * dS[ib][0], e.y * dS[ib][1], e.z * dS[ib][2], e.w * dS[ib][3]};
        if constexpr (HW) dS[ib] += sPB[(w * ST + ib) * 64 + lane];
      }
      if constexpr (HW) {
        // step s: dS[ib] -= W^T d delta (kb = s / ST, ib = s % ST)
        mfma_pipe<2 * ST, 2>([&](int st, uint4& ah, uint4& al) { afrag(sWt, (st % ST) * 2 + st / ST, lane, ah, al); },
                             [&](int st, const uint4& ah, const uint4& al) {
                               dS[st % ST] = mma3(ah, al, dh_[st / ST], dl_[st / ST], dS[st % ST]);
                             });
      } else {
        // step s: kb = s / (2 ST), ib = (s / 2) % ST, operand Qg^T (even s, B = dO) or W^T (odd s)
        mfma_pipe<4 * ST, 2>(
            [&](int st, uint4& ah, uint4& al) {
              afrag((st & 1) ? sWt : sQ, ((st >> 1) % ST) * 2 + st / (2 * ST), lane, ah, al);
            },
            [&](int st, const uint4& ah, const uint4& al) {
              const int kb = st / (2 * ST), ib = (st >> 1) % ST;
              if (st & 1) dS[ib] = mma3(ah, al, dh_[kb], dl_[kb], dS[ib]);
              else dS[ib] = DO_BF16 ? mma2(ah, al, oh[kb], dS[ib]) : mma3(ah, al, oh[kb], ol[kb], dS[ib]);
            });
      }
    }
    __syncthreads();
  }
  // the cotangent entering the group: d h0 (first group), the cotangent leaving group NG-2 (the last
  // group of a grouped pass), or the group's reverse map [Psi | Phi]
  float* dst = nullptr;
  int64_t ld = V;
  if (!real) {
    dst = P.Mg + ((int64_t)bh * P.NG + g) * K * (V + K);
    ld = V + K;
  } else if (g == 0) {
    dst = dh0 ? dh0 + (int64_t)bh * K * V : nullptr;
  } else if (g == P.NG - 1) {
    dst = P.Sg + ((int64_t)bh * P.NG + P.NG - 2) * K * V;
  }
  if (dst) {
#pragma unroll
    for (int ib = 0; ib < ST; ++ib)
#pragma unroll
      for (int j = 0; j < 4; ++j) dst[(int64_t)(16 * ib + 4 * g4 + j) * ld + col] = dS[ib][j];
  }
}

// ===========================================================================
// Pass B of a grouped state pass: `count` serial steps g = g0, g0 + dir, ... of
//   Sg[g + dir] = Phi_g Sg[g] + Psi_g        ([Psi_g | Phi_g] = Mg[g], K x (V + K))
// forward dir = +1 (group-start states), reverse dir = -1 (cotangents leaving each group).
// grid (B*H*V/COLS), block 4 COLS: a wave keeps its 16 columns of S in accumulators, as the state
// passes do; Phi_g (the A operand, rows i, k = j) is split into bf16 hi/lo fragments in LDS.  The
// next step's Phi and Psi are loaded while this step multiplies.  LDS 64 KB.
// ===========================================================================
template <int K, int V>
__global__ __launch_bounds__(state_threads(V)) void state_combine_kernel(GroupPlan P, int BH, int g0, int count,
                                                                            int dir) {
  constexpr int COLS = state_cols(V), NTHR = state_threads(V), NV = V / COLS;
  constexpr int KB = K / 32, ST = K / 16, LD = V + K;
  static_assert((K * K / 4) % NTHR == 0, "staging units per thread");
  constexpr int UP = K * K / 4 / NTHR;  // staging units per thread of Phi
  __shared__ __attribute__((aligned(16))) bf16_t sP[(K / 16) * KB * TILE];
  int bh, vs;
  xcd_map(blockIdx.x, NV, BH, bh, vs);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g4 = lane >> 4;
  const int col = vs * COLS + 16 * w + (lane & 15);
  float4 rP[UP];
  float rPsi[ST][4];
  auto load = [&](int g) {
    const float* m = P.Mg + ((int64_t)bh * P.NG + g) * K * LD;
#pragma unroll
    for (int u = 0; u < UP; ++u) {
      const Unit x = unit<K>(tid + NTHR * u);
      rP[u] = *reinterpret_cast<const float4*>(m + x.row * LD + V + x.k0);
    }
#pragma unroll
    for (int ib = 0; ib < ST; ++ib)
#pragma unroll
      for (int j = 0; j < 4; ++j) rPsi[ib][j] = m[(16 * ib + 4 * g4 + j) * LD + col];
  };
  f32x4 S[ST];
  {
    const float* s0 = P.Sg + ((int64_t)bh * P.NG + g0) * K * V;
#pragma unroll
    for (int ib = 0; ib < ST; ++ib)
#pragma unroll
      for (int j = 0; j < 4; ++j) S[ib][j] = s0[(16 * ib + 4 * g4 + j) * V + col];
  }
  load(g0);
  for (int i = 0; i < count; ++i) {
    const int g = g0 + i * dir;
#pragma unroll
    for (int u = 0; u < UP; ++u) put_unit(sP, unit<K>(tid + NTHR * u).off, rP[u].x, rP[u].y, rP[u].z, rP[u].w);
    f32x4 acc[ST];
#pragma unroll
    for (int ib = 0; ib < ST; ++ib) acc[ib] = f32x4{rPsi[ib][0], rPsi[ib][1], rPsi[ib][2], rPsi[ib][3]};
    __syncthreads();
    if (i + 1 < count) load(g + dir);
    {
      uint4 bh_[KB], bl_[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) bfrag(S[2 * kb], S[2 * kb + 1], bh_[kb], bl_[kb]);
      // step s: ib = s / KB, kb = s % KB
      mfma_pipe<ST * KB, 2>([&](int st, uint4& ah, uint4& al) { afrag(sP, st, lane, ah, al); },
                            [&](int st, const uint4& ah, const uint4& al) {
                              acc[st / KB] = mma3(ah, al, bh_[st % KB], bl_[st % KB], acc[st / KB]);
                            });
    }
    float* dst = P.Sg + ((int64_t)bh * P.NG + g + dir) * K * V;
#pragma unroll
    for (int ib = 0; ib < ST; ++ib) {
      S[ib] = acc[ib];
#pragma unroll
      for (int j = 0; j < 4; ++j) dst[(16 * ib + 4 * g4 + j) * V + col] = acc[ib][j];
    }
    __syncthreads();
  }
}

}  // namespace kdn_state
