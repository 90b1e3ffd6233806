// CCQ read-side cleaning on gfx950: segment walks (K in {64, 128}), forward and backward.
//
// Mathematics (reference ccq/ops/common/fused_read.py:11-25):
//   C_t = h_0 + sum_{j<=t} k_j k_j^T   m_t = m_0 + sum_{j<=t} k_j
//   z_t = C_t^T q_t   s_t = m_t . q_t   corr_t = z_t/pos_t - s_t m_t/pos_t^2 (mean term optional)
//   q_clean_t = q_t - lambda_t corr_t
// Backward, with dz_t = f_t dqc_t, f_t = -lambda_t/pos_t:
//   dlambda_t = -dqc_t . corr_t   ds_t = lambda_t (dqc_t . m_t)/pos_t^2
//   dm_t = -(s_t/pos_t) dz_t + ds_t q_t
//   dq_t = dqc_t + ds_t m_t + C_t dz_t (+ gate: dlogit_t w, dlogit_t = dlambda_t lambda_t (1 - lambda_t))
//   dk_j = E_j k_j + sum_{t>=j} dm_t + dm_T,  E_j = sum_{t>=j} (q_t dz_t^T + dz_t q_t^T) + dC_T + dC_T^T
//   dC_0 = sum_t q_t dz_t^T + dC_T,   dm_0 = sum_t dm_t + dm_T
// C is symmetric (h_0 is taken as symmetric: it is a sum of k k^T in every caller).
//
// Layout of the work.  Both state recurrences are plain sums (C and m forward, E and the dm carry
// backward), so the state at any chunk is a prefix of per-chunk products.  Each (sequence, head) is
// cut into `nseg` time segments of whole 64-token chunks:
//   cs_sum    (forward)  per segment: sum of K^T K and of k          -> segD, segM (saved)
//   cs_fwd    (forward)  walk of one segment from h_0 + earlier segD: q_clean
//   cs_dq     (backward) walk of one segment, recomputing z: dq, the per-token scalars, gate partials
//   cs_gsum   (backward) per segment: sum of Q^T dZ and of dm        -> segG, segDM
//   cs_dk     (backward) reverse walk of one segment from the later segments' totals: dk, dC_0, dm_0
// One workgroup takes one segment; inside it each wavefront owns 16 state columns over all K rows,
// as 16x16 MFMA accumulator tiles in registers, so the state never goes through LDS.  Products that
// read the state take it as their B operand straight from the accumulator layout (lane = column,
// four consecutive rows per 16-lane group), with the contraction slots of the A operand permuted to
// match (two 8-byte LDS reads per lane, frag16_rm_acc).  Row scalars that contract over all of K
// (m . q, the gate logit) are MFMAs against broadcast operands; per-row dot products over the
// columns (dqc . corr, dqc . m) are summed within a wave by DPP and across waves through LDS.
// Every product keeps ~16 significant bits: fp32 operands enter as hi/lo bf16 pairs, q and k are
// exact.  Chunk operands are prefetched into registers one chunk ahead and staged into LDS after
// the chunk's last read; results are staged in LDS and leave as whole 16-byte row pieces after the
// prefetch has been waited for (a single in-order counter covers loads and stores, so a store
// issued before a load would hold the load's wait).
#include "ccq_tile.h"
#include "ccq_walk_args.h"

namespace ccq {

namespace {

constexpr int SB = 64;  // tokens per chunk

__device__ __forceinline__ float seg_pos(int t, int off) {
  const float p = (float)(t + 1 + off);
  return p < 1.f ? 1.f : p;
}

__device__ __forceinline__ bf16x8 ones8_() {
  bf16x8 v;
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (bf16)1.f;
  return v;
}

// A operand of mfma16 (row r = lane % 16) whose contraction slots follow the accumulator layout of
// two 16-row C tiles: lane group g, slot j -> k = 4 g + j (j < 4) and 16 + 4 g + (j - 4) (j >= 4).
// Element (r, k) at p[r * ld + k]: two 8-byte reads.
__device__ __forceinline__ bf16x8 frag16_rm_acc(const bf16* p, int ld) {
  const int l = lane_id();
  const bf16* q = p + (l & 15) * ld + 4 * (l >> 4);
  const bf16x4 a = *(const bf16x4*)q, b = *(const bf16x4*)(q + 16);
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Two fp32 values as packed bf16 hi/lo pairs: hi = the upper 16 bits (truncation), lo = the rest
// rounded to bf16.  hi + lo keeps ~16 significant bits; six VALU operations per pair.
__device__ __forceinline__ void split_pair(float x0, float x1, unsigned& hi, unsigned& lo) {
  const unsigned b0 = __builtin_bit_cast(unsigned, x0), b1 = __builtin_bit_cast(unsigned, x1);
  hi = __builtin_amdgcn_perm(b1, b0, 0x07060302u);
  const float r0 = x0 - __builtin_bit_cast(float, b0 & 0xffff0000u);
  const float r1 = x1 - __builtin_bit_cast(float, b1 & 0xffff0000u);
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  lo = __builtin_bit_cast(unsigned, bf16x2_t{(bf16)r0, (bf16)r1});
}

// B operand (hi/lo) of a 32-deep contraction step from two accumulator tiles holding rows
// [k0, k0 + 16) and [k0 + 16, k0 + 32): slot order of frag16_rm_acc.
__device__ __forceinline__ void acc_pair_split(const f32x4& t0, const f32x4& t1, bf16x8& hi, bf16x8& lo) {
  unsigned h0, h1, h2, h3, o0, o1, o2, o3;
  split_pair(t0[0], t0[1], h0, o0);
  split_pair(t0[2], t0[3], h1, o1);
  split_pair(t1[0], t1[1], h2, o2);
  split_pair(t1[2], t1[3], h3, o3);
  hi = __builtin_bit_cast(bf16x8, u32x4{h0, h1, h2, h3});
  lo = __builtin_bit_cast(bf16x8, u32x4{o0, o1, o2, o3});
}

// Four fp32 values as packed hi/lo bf16x4 (for staged rows).
__device__ __forceinline__ void split4(const f32x4& v, bf16x4& hi, bf16x4& lo) {
  unsigned h0, h1, o0, o1;
  split_pair(v[0], v[1], h0, o0);
  split_pair(v[2], v[3], h1, o1);
  hi = __builtin_bit_cast(bf16x4, u32x2{h0, h1});
  lo = __builtin_bit_cast(bf16x4, u32x2{o0, o1});
}

// Lower-triangular (inclusive) ones as the A operand of mfma16: row t = 16 tt + lane % 16,
// contraction slots s = 32 ss + 8 (lane / 16) + j.
__device__ __forceinline__ bf16x8 tril16(int tt, int ss) {
  const int l = lane_id(), t = 16 * tt + (l & 15), s = 32 * ss + 8 * (l >> 4);
  bf16x8 v;
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = (s + j <= t) ? (bf16)1.f : (bf16)0.f;
  return v;
}

// The lower-triangular ones fragments a (row tile tt, contraction step ss) pair needs: all ones
// below the diagonal block, tril16(0, 0) for even tt and tril16(1, 0) for odd tt on it (the
// diagonal pattern repeats every 32 rows).
struct Tril {
  bf16x8 even, odd, ones;
  __device__ __forceinline__ void init() {
    even = tril16(0, 0);
    odd = tril16(1, 0);
    ones = ones8_();
  }
  __device__ __forceinline__ bf16x8 at(int tt, int ss) const {
    // selects between values (a conditional between the members would take their addresses)
    const u32x4 e = __builtin_bit_cast(u32x4, even), o = __builtin_bit_cast(u32x4, odd);
    const u32x4 n = __builtin_bit_cast(u32x4, ones);
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = ss < (tt >> 1) ? n[i] : ((tt & 1) ? o[i] : e[i]);
    return __builtin_bit_cast(bf16x8, r);
  }
};

// Causal score tile e (0..9) as (t tile, s tile): (0,0) (1,0) (1,1) (2,0) (2,1) (2,2) (3,0) ...
__device__ __forceinline__ int tile_t(int e) { return e < 1 ? 0 : e < 3 ? 1 : e < 6 ? 2 : 3; }
__device__ __forceinline__ int tile_s(int e) { return e - tile_t(e) * (tile_t(e) + 1) / 2; }

// Causal score tile (accumulator of A = K rows 16 J.., B = Q or dZ rows 16 I..: lane = t column,
// rows s) into LDS transposed, as hi/lo bf16: element (t, s) at [16 I + t][16 J + s] of the hi
// plane at p and of the lo plane at p + plane.  `uoff` (the tile's offset, wave-uniform) passes
// through an empty asm so that the per-tile addresses are formed where they are used, not hoisted
// out of the chunk loop into registers that would then be spilled.
__device__ __forceinline__ void score_to_lds(const f32x4& acc, bf16* p, int plane, int ld, int uoff) {
  asm volatile("" : "+s"(uoff));
  bf16x4 hh, ll;
  split4(acc, hh, ll);
  const int e = uoff + (lane_id() & 15) * ld + 4 * (lane_id() >> 4);
  *(bf16x4*)(p + e) = hh;
  *(bf16x4*)(p + plane + e) = ll;
}

// State columns per workgroup of the segment sums (one 16-column tile per wavefront) and column
// blocks per (sequence, head): 64-column blocks, so that K = 128 runs two 4-wave workgroups per
// (sequence, head, segment) -- two resident per CU -- instead of one 8-wave workgroup.  The walks
// (K in {64, 128}) keep all K columns in one workgroup.
template <int K>
struct SegCols {
  static constexpr int CW = K > 64 ? 64 : K, NCB = K / CW, NW = CW / 16, NT = 64 * NW;
};

// One segment of one (sequence, head) and one column block: chunks [cb, ce) of the sequence's nc
// chunks, state columns [cbase, cbase + CW).
struct SegUnit {
  int unit, seg, cbase, n, h, len, nc, cb, ce, gc0;
  long bos, hb, rs;
};

// NCB column blocks per (sequence, head, segment): 1 for the walks, SegCols<K>::NCB for the sums.
template <int K, int NCB = 1>
__device__ __forceinline__ SegUnit seg_unit(const WalkArgs& a) {
  SegUnit u;
  int sub;
  xcd_map(blockIdx.x, a.nseg * NCB, a.N * a.H, u.unit, sub);
  u.seg = sub / NCB;
  u.cbase = (sub % NCB) * (K / NCB);
  u.n = u.unit / a.H;
  u.h = u.unit % a.H;
  seq_bounds(a.cu, u.n, a.T, u.bos, u.len);
  u.nc = (u.len + SB - 1) / SB;
  const int per = (u.nc + a.nseg - 1) / a.nseg;
  u.cb = min(u.nc, u.seg * per);
  u.ce = min(u.nc, u.cb + per);
  u.gc0 = a.cu ? a.chunk_off[u.n] : u.n * a.NT;
  u.rs = (long)a.H * K;
  u.hb = (u.bos * a.H + u.h) * K;
  return u;
}

// Buffer resource over rows [0, L) of a token-major tensor (row stride rs elements, row_elems
// elements used per row, esize bytes each) from p: accesses to rows at or beyond L -- or to anything,
// when p is null -- are dropped by the hardware (stores) or read as zero (loads).  Every thread then
// issues the same memory operations whatever L is, so the compiler's wait counts follow one fixed
// sequence and a wait for a load never covers a younger store.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const void* p, long rs, int L, int row_elems,
                                                            int esize) {
  return buf_rsrc(p, (p != nullptr && L > 0) ? (int)(((long)(L - 1) * rs + row_elems) * esize) : 0);
}

// One thread's pieces of a SB x K fp32 tile in the piece mapping of RowsF32<K, SB, NT> (16 consecutive
// lanes per 256-byte row segment): read from LDS, written to HBM as fp32 and / or bf16 rows.
template <int K, int NT>
struct TileOut {
  static constexpr int VPR = K / 4, N = SB * VPR / NT;
  static_assert((SB * VPR) % NT == 0, "whole passes");
  f32x4 v[N];
  __device__ __forceinline__ void read(const float* src, int ld, int tid) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = tid + j * NT;
      v[j] = *(const f32x4*)(src + (idx / VPR) * ld + (idx % VPR) * 4);
    }
  }
  // w32 / w16 (uniform over the launch) select the outputs asked for: a store to an absent output
  // would be dropped by its resource, but it would still take the vector-memory issue slots.
  __device__ __forceinline__ void store(__amdgpu_buffer_rsrc_t r32, __amdgpu_buffer_rsrc_t r16, long rs,
                                        int tid, bool w32, bool w16) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = tid + j * NT;
      const int e = (int)((idx / VPR) * rs + (idx % VPR) * 4);
      if (w32) __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[j]), r32, e * 4, 0, 0);
      const bf16x4 b = bf16x4{(bf16)v[j][0], (bf16)v[j][1], (bf16)v[j][2], (bf16)v[j][3]};
      if (w16) __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, b), r16, e * 2, 0, 0);
    }
  }
};

// fp32 rows of a chunk into registers through a rows_rsrc resource (zero past the chunk or when the
// tensor is absent), in the piece mapping of TileOut.
template <int K, int NT>
struct TileIn {
  static constexpr int VPR = K / 4, N = SB * VPR / NT;
  f32x4 v[N];
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, long rs, int tid) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = tid + j * NT;
      const int e = (int)((idx / VPR) * rs + (idx % VPR) * 4);
      v[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, e * 4, 0, 0));
    }
  }
  __device__ __forceinline__ void store(float* dst, int ld, int tid) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = tid + j * NT;
      *(f32x4*)(dst + (idx / VPR) * ld + (idx % VPR) * 4) = v[j];
    }
  }
  // zeros over the pieces store() writes
  __device__ __forceinline__ void zero(float* dst, int ld, int tid) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = tid + j * NT;
      *(f32x4*)(dst + (idx / VPR) * ld + (idx % VPR) * 4) = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
};

// Sum of the segment totals tot[unit][s] for s in [s0, s1) into the lane's accumulator tiles
// (rows 16 kt + g4 + i, column col), optionally plus the transposed tiles (tot[.][col][k]).
template <int K, bool TRANS>
__device__ __forceinline__ void add_seg_tiles(f32x4 (&X)[K / 16], const float* tot, long unit, int nseg, int s0,
                                              int s1, int col, int g4) {
  for (int s = s0; s < s1; ++s) {
    const float* p = tot + ((long)unit * nseg + s) * K * K;
#pragma unroll
    for (int kt = 0; kt < K / 16; ++kt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) X[kt][i] += p[(long)(16 * kt + g4 + i) * K + col];
      if (TRANS) X[kt] += *(const f32x4*)(p + (long)col * K + 16 * kt + g4);
    }
  }
}

}  // namespace

// ===========================================================================
// cs_sum: grid N*H*nseg*NCB, CW/16 waves.  segD[:, cols] = sum over the segment's chunks of
// K^T K[:, cols], segM[cols] = sum of k (every workgroup writes its totals, zero for an empty
// segment).  Two chunks in flight.
// ===========================================================================
template <int K>
__global__ __launch_bounds__(SegCols<K>::NT) void cs_sum_kernel(const WalkArgs a) {
  constexpr int NT = SegCols<K>::NT, LDK = K + 16, NKT = K / 16;
  __shared__ __attribute__((aligned(16))) bf16 sK[2][SB * LDK];
  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(wave_id()), l = lane_id();
  const SegUnit u = seg_unit<K, SegCols<K>::NCB>(a);
  const int c0 = u.cbase + 16 * w, col = c0 + (l & 15), g4 = 4 * (l >> 4);
  auto chunk_len = [&](int c) { return min(SB, u.len - c * SB); };
  f32x4 D[NKT];
#pragma unroll
  for (int kt = 0; kt < NKT; ++kt) D[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float msum = 0.f;
  RowsBf16<K, SB, NT> p0, p1;
  auto kptr = [&](int c) { return (const bf16*)a.k + u.hb + (long)c * SB * u.rs; };
  const int nloc = u.ce - u.cb;
  // past the end the last chunk is loaded and staged again (into the idle buffer): every pass issues
  // the same memory operations
  auto cl = [&](int i) { return min(u.cb + i, u.ce - 1); };
  if (nloc > 0) {
    p0.load(kptr(cl(0)), u.rs, chunk_len(cl(0)), tid);
    p1.load(kptr(cl(1)), u.rs, chunk_len(cl(1)), tid);
    p0.store(sK[0], LDK, chunk_len(cl(0)), tid);
  }
  __syncthreads();
  auto step = [&](int i, RowsBf16<K, SB, NT>& cur, RowsBf16<K, SB, NT>& nxt) {
    // chunk cb + i is in buffer i & 1; `cur` is free (staged), `nxt` holds chunk cb + i + 1
    const bf16* Kc = sK[i & 1];
    cur.load(kptr(cl(i + 2)), u.rs, chunk_len(cl(i + 2)), tid);
    bf16x8 kcol[2];
#pragma unroll
    for (int ss = 0; ss < 2; ++ss) kcol[ss] = frag16_tr(Kc + 32 * ss * LDK + c0, LDK);
    f32x4 tot = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ss = 0; ss < 2; ++ss) {
      tot = mfma16(tril16(3, ss), kcol[ss], tot);
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt) D[kt] = mfma16(frag16_tr(Kc + 32 * ss * LDK + 16 * kt, LDK), kcol[ss], D[kt]);
    }
    msum += __shfl(tot[3], 48 + (l & 15));
    nxt.store(sK[(i + 1) & 1], LDK, chunk_len(cl(i + 1)), tid);
    __syncthreads();
  };
  int i = 0;
  for (; i + 1 < nloc; i += 2) {
    step(i, p0, p1);
    step(i + 1, p1, p0);
  }
  if (i < nloc) step(i, p0, p1);
  float* dst = a.segD + ((long)u.unit * a.nseg + u.seg) * K * K;
#pragma unroll
  for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
    for (int r = 0; r < 4; ++r) dst[(long)(16 * kt + g4 + r) * K + col] = D[kt][r];
  if (l < 16) a.segM[((long)u.unit * a.nseg + u.seg) * K + col] = msum;
}

// ===========================================================================
// cs_fwd: grid N*H*nseg, K/16 waves (one per 16 state columns).  Per chunk:
//   scores   A = (Q K^T) o M: 10 causal 16x16 tiles spread over the waves, to LDS as hi/lo bf16
//   scalars  s_t = m_prev . q_t + sum_s A[t][s], the gate logit w . q_t: MFMAs against broadcast
//            operands, one 16-row tile per wave of the last four
//   per wave Z[:, cols] = Q C_prev[:, cols] + A K[:, cols]; running key sums (lower-triangular ones
//            times K[:, cols]); q_clean to LDS; C[:, cols] += K^T K[:, cols]
//   all      chunk c+1 from registers into the other LDS buffers; q_clean rows to registers, to HBM
//            during the next chunk's products
// Outputs: q_clean (bf16 and/or fp32), the gate's lambda, C_T and m_T (last segment).
// ===========================================================================
template <int K, bool MEAN, bool GATE>
__global__ __launch_bounds__(K * 4) void cs_fwd_kernel(const WalkArgs a) {
  static_assert(K <= 128, "segment walks hold all K columns of a (sequence, head) in one workgroup");
  constexpr int NW = K / 16, NT = 64 * NW;
  // row pitch of the q / k tiles: K + 8 bf16 (a pitch of 4 banks mod 32 spreads the 16 rows of a
  // fragment read; measured faster here than K + 16)
  constexpr int LDK = K + 8, LDA = SB + 16, LDO = K + 4;
  constexpr int NKS = K / 32, NKT = K / 16;
  __shared__ __attribute__((aligned(16))) bf16 sQ[2][SB * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sK[2][SB * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sA[2 * SB * LDA];  // scores A[t][s] (s <= t): hi, lo planes
  bf16* const sAh = sA;
  bf16* const sAl = sA + SB * LDA;
  __shared__ __attribute__((aligned(16))) float sO[SB * LDO];   // q_clean rows
  __shared__ __attribute__((aligned(16))) bf16 sMW[2][4 * LDK];  // rows: m hi, m lo, gate w hi, lo
  __shared__ __attribute__((aligned(16))) float sS[SB];          // s_t, then s_t / pos_t^2
  __shared__ __attribute__((aligned(16))) float sLam[SB];        // lambda_t
  __shared__ __attribute__((aligned(16))) float sIp[SB];         // 1 / pos_t
  __shared__ __attribute__((aligned(16))) float sLamIn[2][SB];   // given lambda, by buffer

  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(wave_id()), l = lane_id();
  const SegUnit u = seg_unit<K>(a);
  const bool last = u.seg == a.nseg - 1;
  if (u.cb >= u.ce && !last) return;
  const int c0 = 16 * w, col = c0 + (l & 15), g4 = 4 * (l >> 4);
  auto chunk_len = [&](int c) { return min(SB, u.len - c * SB); };
  Tril tri;
  tri.init();

  // state at the segment start: h_0 + the earlier segments' K^T K; the lane's column of the key sum
  f32x4 C[NKT];
#pragma unroll
  for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
    for (int i = 0; i < 4; ++i) C[kt][i] = a.h0 ? a.h0[((long)u.unit * K + 16 * kt + g4 + i) * K + col] : 0.f;
  add_seg_tiles<K, false>(C, a.segD, u.unit, a.nseg, 0, u.seg, col, g4);
  float mcol = 0.f;
  if (MEAN) {
    mcol = a.m0 ? a.m0[(long)u.unit * K + col] : 0.f;
    for (int s = 0; s < u.seg; ++s) mcol += a.segM[((long)u.unit * a.nseg + s) * K + col];
  }
#pragma unroll
  for (int kt = 0; kt < NKT; ++kt) settle(C[kt]);
  settle(mcol);

  // LDS set-up: scores above the diagonal tiles stay zero; gate rows of both buffers; key sums
  for (int i = tid; i < SB * LDA; i += NT) {
    sAh[i] = (bf16)0.f;
    sAl[i] = (bf16)0.f;
  }
  for (int i = tid; i < 2 * K; i += NT) {
    const int r = i / K, cc = i % K;
    bf16 hh = (bf16)0.f, ll = (bf16)0.f;
    if (GATE) split2(a.gate_w[(long)u.h * K + cc], hh, ll);
    sMW[0][(2 + r) * LDK + cc] = r == 0 ? hh : ll;
    sMW[1][(2 + r) * LDK + cc] = r == 0 ? hh : ll;
  }
  auto put_m = [&](int b) {
    if (l < 16) {
      bf16 x, y;
      split2(mcol, x, y);
      sMW[b][col] = x;
      sMW[b][LDK + col] = y;
    }
  };
  if (MEAN) put_m(u.cb & 1);

  RowsBf16<K, SB, NT> pq, pk;
  float plam = 0.f;
  // chunk loads and stages: unconditional (past the end the last chunk again, into the idle buffer)
  auto load = [&](int c) {
    const int L = chunk_len(c);
    const long off = u.hb + (long)c * SB * u.rs;
    pk.load((const bf16*)a.k + off, u.rs, L, tid);
    pq.load((const bf16*)a.q + off, u.rs, L, tid);
    if (!GATE) plam = a.lam[(u.bos + (long)c * SB + min(tid & (SB - 1), L - 1)) * a.H + u.h];
  };
  auto stage = [&](int c, int b) {
    const int L = chunk_len(c);
    pk.store(sK[b], LDK, L, tid);
    pq.store(sQ[b], LDK, L, tid);
    if (!GATE && tid < SB) sLamIn[b][tid] = tid < L ? plam : 0.f;
  };
  if (u.cb < u.ce) {
    load(u.cb);
    stage(u.cb, u.cb & 1);
    load(min(u.cb + 1, u.ce - 1));
  }
  __syncthreads();
  // q_clean rows and gate values of a chunk, held in registers from the end of its pass to the
  // next pass's stores (which then overlap that pass's products)
  TileOut<K, NT> out;
  float lamo = 0.f;
  auto put_out = [&](int pc) {
    const int L = chunk_len(pc), t0 = pc * SB;
    const long ob = u.hb + (long)t0 * u.rs;
    out.store(rows_rsrc(a.qc32 ? a.qc32 + ob : nullptr, u.rs, L, K, 4),
              rows_rsrc(a.qc ? (const bf16*)a.qc + ob : nullptr, u.rs, L, K, 2), u.rs, tid, a.qc32 != nullptr,
              a.qc != nullptr);
    if (GATE && w == 0 && a.lam_out) {
      // the chunk's SB gate values from wave 0 (row = lane)
      static_assert(SB == 64, "per-token outputs fit wave 0");
      const __amdgpu_buffer_rsrc_t rl = rows_rsrc(a.lam_out + (u.bos + t0) * a.H + u.h, a.H, L, 1, 4);
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, lamo), rl, tid * a.H * 4, 0, 0);
    }
  };

  float gbias = GATE ? a.gate_b[u.h] : 0.f;
  settle(gbias);
  for (int c = u.cb; c < u.ce; ++c) {
    const int b = c & 1, L = chunk_len(c), t0 = c * SB;
    const bf16* Qc = sQ[b];
    const bf16* Kc = sK[b];
    bf16x8 kcol[2];
#pragma unroll
    for (int ss = 0; ss < 2; ++ss) kcol[ss] = frag16_tr(Kc + 32 * ss * LDK + c0, LDK);

    // ---- scores (tiles w, w + NW, w + 2 NW) and row scalars (t tile w - (NW - 4))
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int e = w + j * NW;
      if (e < 10) {
        const int I = tile_t(e), J = tile_s(e);
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks)
          acc = mfma16(frag16_rm(Kc + 16 * J * LDK + 32 * ks, LDK), frag16_rm(Qc + 16 * I * LDK + 32 * ks, LDK), acc);
        if (I == J) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (g4 + i > (l & 15)) acc[i] = 0.f;
        }
        score_to_lds(acc, sA, SB * LDA, LDA, 16 * I * LDA + 16 * J);
      }
    }
    if (w >= NW - 4) {
      const int tt = w - (NW - 4), tb = 16 * tt + g4;
      f32x4 sv = f32x4{0.f, 0.f, 0.f, 0.f}, lg = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const bf16x8 qf = frag16_rm(Qc + 16 * tt * LDK + 32 * ks, LDK);
        if (MEAN) {
          sv = mfma16(qf, frag16_rm(sMW[b] + 32 * ks, 0), sv);
          sv = mfma16(qf, frag16_rm(sMW[b] + LDK + 32 * ks, 0), sv);
        }
        if (GATE) {
          lg = mfma16(qf, frag16_rm(sMW[b] + 2 * LDK + 32 * ks, 0), lg);
          lg = mfma16(qf, frag16_rm(sMW[b] + 3 * LDK + 32 * ks, 0), lg);
        }
      }
      // (the score row sums join s_t after the barrier: other waves write those tiles)
      if ((l & 15) == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = tb + i;
          float lam;
          if (GATE) lam = t < L ? __builtin_amdgcn_rcpf(1.f + __expf(-(lg[i] + gbias))) : 0.f;
          else lam = sLamIn[b][t];
          sLam[t] = lam;
          sS[t] = sv[i];
          sIp[t] = __builtin_amdgcn_rcpf(seg_pos(t0 + t, a.pos_off));
        }
      }
    }
    __syncthreads();
    if (c > u.cb) put_out(c - 1);
    if (MEAN) {
      if (w >= NW - 4) {
        const int tt = w - (NW - 4), tb = 16 * tt + g4;
        f32x4 rsum = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ss = 0; ss < 2; ++ss) {
          if (ss <= (tt >> 1)) {
            rsum = mfma16(frag16_rm(sAh + 16 * tt * LDA + 32 * ss, LDA), ones8_(), rsum);
            rsum = mfma16(frag16_rm(sAl + 16 * tt * LDA + 32 * ss, LDA), ones8_(), rsum);
          }
        }
        if ((l & 15) == 0) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float ip = sIp[tb + i];
            sS[tb + i] = (sS[tb + i] + rsum[i]) * ip * ip;
          }
        }
      }
      __syncthreads();
    }

    // ---- per wave: Z[:, cols] = Q C_prev[:, cols] + A K[:, cols]; key sums; q_clean to LDS.  The
    // state's hi/lo B operands are formed once per chunk; then one 16-row tile at a time (a runtime
    // loop keeps the live registers few), hi and lo products in separate accumulators
    bf16x8 chh[NKS], chl[NKS];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) acc_pair_split(C[2 * ks], C[2 * ks + 1], chh[ks], chl[ks]);
    f32x4 cum = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int tt = 0; tt < 4; ++tt) {
      f32x4 zh = f32x4{0.f, 0.f, 0.f, 0.f}, zl = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const bf16x8 qa = frag16_rm_acc(Qc + 16 * tt * LDK + 32 * ks, LDK);
        zh = mfma16(qa, chh[ks], zh);
        zl = mfma16(qa, chl[ks], zl);
      }
      cum = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ss = 0; ss < 2; ++ss) {
        if (ss <= (tt >> 1)) {
          zh = mfma16(frag16_rm(sAh + 16 * tt * LDA + 32 * ss, LDA), kcol[ss], zh);
          zl = mfma16(frag16_rm(sAl + 16 * tt * LDA + 32 * ss, LDA), kcol[ss], zl);
          if (MEAN) cum = mfma16(tri.at(tt, ss), kcol[ss], cum);
        }
      }
      const int tb = 16 * tt + g4;
      const f32x4 ipv = *(const f32x4*)(sIp + tb), lamv = *(const f32x4*)(sLam + tb);
      f32x4 sv = f32x4{0.f, 0.f, 0.f, 0.f};
      if (MEAN) sv = *(const f32x4*)(sS + tb);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float corr = (zh[i] + zl[i]) * ipv[i];
        if (MEAN) corr -= sv[i] * (mcol + cum[i]);
        sO[(tb + i) * LDO + col] = (float)Qc[(tb + i) * LDK + col] - lamv[i] * corr;
      }
    }
    // key-sum total of the chunk: row 63 of the running sums (rows past the chunk hold k = 0)
    if (MEAN) mcol += __shfl(cum[3], 48 + (l & 15));

    // ---- state update C[:, cols] += K^T K[:, cols]
#pragma unroll
    for (int ss = 0; ss < 2; ++ss)
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt) C[kt] = mfma16(frag16_tr(Kc + 32 * ss * LDK + 16 * kt, LDK), kcol[ss], C[kt]);
    if (MEAN) put_m(b ^ 1);
    stage(min(c + 1, u.ce - 1), b ^ 1);
    lamo = sLam[tid & (SB - 1)];  // (rewritten before the next chunk's first barrier)
    __syncthreads();
    // results of chunk c to registers (stored during the next pass); loads of chunk c+2
    out.read(sO, LDO, tid);
    load(min(c + 2, u.ce - 1));
  }
  if (u.cb < u.ce) put_out(u.ce - 1);

  if (last) {
    if (a.h_fin) {
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) a.h_fin[((long)u.unit * K + 16 * kt + g4 + i) * K + col] = C[kt][i];
    }
    if (MEAN && a.m_fin && l < 16) a.m_fin[(long)u.unit * K + col] = mcol;
  }
}

// ===========================================================================
// cs_dq: grid N*H*nseg, K/16 waves; the forward walk again, with the upstream gradient.  The
// backward needs z_t only through dqc_t . z_t = q_t . (C_t dqc_t) (C_t symmetric), so the walk forms
// W'_t = C_t dqc_t alone -- no Q C, no (Q K^T) o M scores -- and dq_t's state term is f_t W'_t.
// Per chunk (dQc hi/lo in LDS, staged with the chunk):
//   1  score tiles B = (dQc K^T) o M (10 tiles over the waves)
//   2  per wave and 16-row tile: W' = dQc C + B K and m_t; partial row dots over the wave's columns
//      of q . W' (= dqc . z), dqc . m_t and q . m_t (= s_t); dqc + f W' in place
//   3  wave 0, lane = token: row totals of the partial dots, then dlambda, ds, dlogit and the
//      per-token outputs
//   4  per wave: dq = dqc + f W' + ds m_t (+ dlogit w) in place; gate partials; C, m update
//   5  results to registers, chunk c+1 into LDS (each thread overwrites exactly the pieces it stored)
// The results of chunk c leave during the products of chunk c+1, and the upstream gradient of chunk
// c+1 is loaded during them too: the vector-memory traffic spreads over the pass instead of
// queueing behind one barrier in every workgroup at once.
// ===========================================================================
template <int K, bool MEAN, bool GATE, bool DQ32>
__global__ __launch_bounds__(K * 4) void cs_dq_kernel(const WalkArgs a) {
  static_assert(K <= 128, "segment walks hold all K columns of a (sequence, head) in one workgroup");
  constexpr int NW = K / 16, NT = 64 * NW;
  constexpr int LDK = K + 16, LDA = SB + 16, LDD = K + 4;
  constexpr int NKS = K / 32, NKT = K / 16;
  constexpr int NP = MEAN ? 3 : 1;  // partial row dots per token
  static_assert(NT >= NP * SB, "one thread per row total");
  __shared__ __attribute__((aligned(16))) bf16 sQ[SB * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sK[SB * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sZh[SB * LDK];   // dQc, hi
  __shared__ __attribute__((aligned(16))) bf16 sZl[SB * LDK];
  __shared__ __attribute__((aligned(16))) float sD[SB * LDD];   // dQc, then dQc + f W', then dq
  // score planes: (dQc K^T) o M hi, lo
  __shared__ __attribute__((aligned(16))) bf16 sB[2 * SB * LDA];
  bf16* const sBh = sB;
  bf16* const sBl = sB + SB * LDA;
  __shared__ __attribute__((aligned(16))) float sPart[NW][NP][SB];  // per-wave partial row dots
  __shared__ __attribute__((aligned(16))) float sDs[SB], sDg[SB];  // per token: ds, dlogit
  __shared__ __attribute__((aligned(16))) float sLam[SB], sF[SB], sIp[SB], sGw[K];
  __shared__ __attribute__((aligned(16))) f32x4 sScO[SB];   // per-token scalars of the chunk (out)
  __shared__ __attribute__((aligned(16))) float sDlO[SB];   // dlambda (out)
  __shared__ __attribute__((aligned(16))) float sGp[K + 4];  // gate partials: dW columns, db (out)

  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(wave_id()), l = lane_id();
  const SegUnit u = seg_unit<K>(a);
  if (u.cb >= u.ce) return;
  const int c0 = 16 * w, col = c0 + (l & 15), g4 = 4 * (l >> 4);
  auto chunk_len = [&](int c) { return min(SB, u.len - c * SB); };
  Tril tri;
  tri.init();

  f32x4 C[NKT];
#pragma unroll
  for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
    for (int i = 0; i < 4; ++i) C[kt][i] = a.h0 ? a.h0[((long)u.unit * K + 16 * kt + g4 + i) * K + col] : 0.f;
  add_seg_tiles<K, false>(C, a.segD, u.unit, a.nseg, 0, u.seg, col, g4);
  float mcol = 0.f;
  if (MEAN) {
    mcol = a.m0 ? a.m0[(long)u.unit * K + col] : 0.f;
    for (int s = 0; s < u.seg; ++s) mcol += a.segM[((long)u.unit * a.nseg + s) * K + col];
  }
#pragma unroll
  for (int kt = 0; kt < NKT; ++kt) settle(C[kt]);
  settle(mcol);
  for (int i = tid; i < SB * LDA; i += NT) {
    sBh[i] = (bf16)0.f;
    sBl[i] = (bf16)0.f;
  }
  if (GATE)
    for (int i = tid; i < K; i += NT) sGw[i] = a.gate_w[(long)u.h * K + i];

  RowsBf16<K, SB, NT> pq, pk;
  RowsF32<K, SB, NT> pd;
  constexpr int ND = RowsF32<K, SB, NT>::N, VPR = K / 4;
  float plam = 0.f;
  // chunk loads in two parts, issued at different points of a pass so that the vector-memory
  // traffic of all workgroups spreads over the pass: k, q, lambda; the upstream gradient
  auto load_a = [&](int c) {
    const int L = chunk_len(c);
    const long off = u.hb + (long)c * SB * u.rs;
    pk.load((const bf16*)a.k + off, u.rs, L, tid);
    pq.load((const bf16*)a.q + off, u.rs, L, tid);
    plam = a.lam_used[(u.bos + (long)c * SB + min(tid & (SB - 1), L - 1)) * a.H + u.h];
  };
  auto load_b = [&](int c) {
    const int L = chunk_len(c);
    const long off = u.hb + (long)c * SB * u.rs;
    // (the upstream gradient's dtype is a template parameter: one load sequence)
    if (DQ32) pd.load(a.dqc32 + off, u.rs, L, tid);
    else pd.load(nullptr, (const bf16*)a.dqc16 + off, u.rs, L, tid);
  };
  auto stage = [&](int c) {
    const int L = chunk_len(c), t0 = c * SB;
    pk.store(sK, LDK, L, tid);
    pq.store(sQ, LDK, L, tid);
    pd.store(sD, LDD, L, tid);
#pragma unroll
    for (int j = 0; j < ND; ++j) {
      const int idx = tid + j * NT, r = idx / VPR, cc = (idx % VPR) * 4;
      bf16x4 hh, ll;
      split4(pd.v[j], hh, ll);
      *(bf16x4*)(sZh + r * LDK + cc) = hh;
      *(bf16x4*)(sZl + r * LDK + cc) = ll;
    }
    if (tid < SB) {
      const bool ok = tid < L;
      const float ip = __builtin_amdgcn_rcpf(seg_pos(t0 + tid, a.pos_off));
      sLam[tid] = ok ? plam : 0.f;
      sF[tid] = ok ? -plam * ip : 0.f;
      sIp[tid] = ip;
    }
  };
  // results of a chunk, held in registers from the end of its pass to the next pass's stores
  TileOut<K, NT> out;
  f32x4 sco = f32x4{0.f, 0.f, 0.f, 0.f}, gpo = f32x4{0.f, 0.f, 0.f, 0.f};
  float dlo = 0.f, dbo = 0.f;
  // the stores of chunk pc (the previous pass's): dq rows, and the per-token outputs from wave 0
  // (the chunk's SB rows are its 64 lanes)
  auto put_out = [&](int pc) {
    const int L = chunk_len(pc), t0 = pc * SB;
    const long ob = u.hb + (long)t0 * u.rs, tb0 = (u.bos + t0) * a.H + u.h;
    out.store(rows_rsrc(a.dq32 ? a.dq32 + ob : nullptr, u.rs, L, K, 4),
              rows_rsrc(a.dq ? (const bf16*)a.dq + ob : nullptr, u.rs, L, K, 2), u.rs, tid, a.dq32 != nullptr,
              a.dq != nullptr);
    if (w == 0) {
      static_assert(SB == 64 && K / 4 <= 64, "per-token outputs fit wave 0");
      constexpr int kPast = 0x7ffffff0;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, sco),
                                             rows_rsrc(a.sc + tb0 * 4, a.H * 4, L, 4, 4), tid * a.H * 16, 0, 0);
      if (!GATE && a.dlam)
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, dlo), rows_rsrc(a.dlam + tb0, a.H, L, 1, 4),
                                              tid * a.H * 4, 0, 0);
      if (GATE) {
        const long gi = (long)(u.gc0 + pc) * a.H + u.h;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, gpo), buf_rsrc(a.dw_part + gi * K, K * 4),
                                               tid < K / 4 ? tid * 16 : kPast, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, dbo), buf_rsrc(a.db_part + gi, 4),
                                              tid == 0 ? 0 : kPast, 0, 0);
      }
    }
  };
  // chunk loads and stages: unconditional (past the end the last chunk again)
  load_a(u.cb);
  load_b(u.cb);
  stage(u.cb);
  load_a(min(u.cb + 1, u.ce - 1));
  __syncthreads();

  for (int c = u.cb; c < u.ce; ++c) {
    const int L = chunk_len(c), t0 = c * SB;
    bf16x8 kcol[2];
#pragma unroll
    for (int ss = 0; ss < 2; ++ss) kcol[ss] = frag16_tr(sK + 32 * ss * LDK + c0, LDK);

    // ---- 1: score tiles
#pragma unroll
    for (int j = 0; j < (10 + NW - 1) / NW; ++j) {
      const int e = w + j * NW;
      if (e < 10) {
        const int I = tile_t(e), J = tile_s(e);
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          const bf16x8 kf = frag16_rm(sK + 16 * J * LDK + 32 * ks, LDK);
          acc = mfma16(kf, frag16_rm(sZh + 16 * I * LDK + 32 * ks, LDK), acc);
          acc = mfma16(kf, frag16_rm(sZl + 16 * I * LDK + 32 * ks, LDK), acc);
        }
        if (I == J) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (g4 + i > (l & 15)) acc[i] = 0.f;
        }
        score_to_lds(acc, sB, SB * LDA, LDA, 16 * I * LDA + 16 * J);
      }
    }
    __syncthreads();
    // the previous chunk's results leave while this chunk's products run
    if (c > u.cb) put_out(c - 1);

    // ---- 2: per wave, one 16-row tile at a time (the state's hi/lo B operands formed once)
    bf16x8 chh[NKS], chl[NKS];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) acc_pair_split(C[2 * ks], C[2 * ks + 1], chh[ks], chl[ks]);
#pragma unroll 1
    for (int tt = 0; tt < 4; ++tt) {
      // three independent accumulator chains: hi x hi, lo x hi, hi x lo
      f32x4 wh = f32x4{0.f, 0.f, 0.f, 0.f}, wl = f32x4{0.f, 0.f, 0.f, 0.f}, wm = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const bf16x8 da = frag16_rm_acc(sZh + 16 * tt * LDK + 32 * ks, LDK);
        const bf16x8 dl = frag16_rm_acc(sZl + 16 * tt * LDK + 32 * ks, LDK);
        wh = mfma16(da, chh[ks], wh);
        wl = mfma16(dl, chh[ks], wl);
        wm = mfma16(da, chl[ks], wm);
      }
      f32x4 cum = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ss = 0; ss < 2; ++ss) {
        if (ss <= (tt >> 1)) {
          wh = mfma16(frag16_rm(sBh + 16 * tt * LDA + 32 * ss, LDA), kcol[ss], wh);
          wl = mfma16(frag16_rm(sBl + 16 * tt * LDA + 32 * ss, LDA), kcol[ss], wl);
          if (MEAN) cum = mfma16(tri.at(tt, ss), kcol[ss], cum);
        }
      }
      const int tb = 16 * tt + g4;
      const f32x4 fv = *(const f32x4*)(sF + tb);
      f32x4 p1, p2, p3;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float* pd_ = sD + (tb + i) * LDD + col;
        const float dqc = *pd_;
        const float qv = (float)sQ[(tb + i) * LDK + col];
        const float wv = wh[i] + (wl[i] + wm[i]);
        const float mt = mcol + cum[i];
        p1[i] = qv * wv;
        p2[i] = dqc * mt;
        p3[i] = qv * mt;
        *pd_ = dqc + fv[i] * wv;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p1[i] = row16_sum(p1[i]);
        if (MEAN) {
          p2[i] = row16_sum(p2[i]);
          p3[i] = row16_sum(p3[i]);
        }
      }
      if ((l & 15) == 0) {
        *(f32x4*)(&sPart[w][0][tb]) = p1;
        if (MEAN) {
          *(f32x4*)(&sPart[w][MEAN ? 1 : 0][tb]) = p2;
          *(f32x4*)(&sPart[w][MEAN ? 2 : 0][tb]) = p3;
        }
      }
    }
    // the upstream gradient of chunk c+1 (its registers were staged at the end of the last pass)
    load_b(min(c + 1, u.ce - 1));
    __syncthreads();
    // ---- 3: per token (wave 0, lane = token): the row totals dqc . z, dqc . m, s and from them
    // dlambda, ds, dlogit; the per-token outputs; the gate bias partial
    if (w == 0) {
      const int t = l;
      float t0 = 0.f, t1 = 0.f, sv = 0.f;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) {
        t0 += sPart[ww][0][t];
        if (MEAN) {
          t1 += sPart[ww][MEAN ? 1 : 0][t];
          sv += sPart[ww][MEAN ? 2 : 0][t];
        }
      }
      const float lam = sLam[t], ip = sIp[t];
      // dqc . corr = (dqc . z)/pos - s (dqc . m)/pos^2
      float dcorr = t0 * ip;
      if (MEAN) dcorr -= sv * ip * ip * t1;
      const float dlam = t < L ? -dcorr : 0.f;
      const float ds = MEAN ? lam * t1 * ip * ip : 0.f;
      const float dlogit = dlam * lam * (1.f - lam);
      sDs[t] = ds;
      sDg[t] = dlogit;
      sScO[t] = f32x4{sF[t], ds, GATE ? dlogit : dlam, MEAN ? -sv * ip : 0.f};
      sDlO[t] = GATE ? dlogit : dlam;
      if (GATE) {
        // wave sum: within each 16-lane row by DPP, then the four row sums
        const float tot = wave_total(dlogit);
        if (l == 0) sGp[K] = tot;
      }
    }
    __syncthreads();

    // ---- 4: dq (+ ds m_t, + dlogit w), gate column partials, state update
    float gsum = 0.f;
    const float gwc = GATE ? sGw[col] : 0.f;
    f32x4 cum = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      cum = f32x4{0.f, 0.f, 0.f, 0.f};
      if (MEAN) {
#pragma unroll
        for (int ss = 0; ss < 2; ++ss)
          if (ss <= (tt >> 1)) cum = mfma16(tri.at(tt, ss), kcol[ss], cum);
      }
      const int tb = 16 * tt + g4;
      const f32x4 dsv = *(const f32x4*)(sDs + tb);
      f32x4 dgv = f32x4{0.f, 0.f, 0.f, 0.f};
      if (GATE) dgv = *(const f32x4*)(sDg + tb);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float* pd_ = sD + (tb + i) * LDD + col;
        float dq = *pd_;
        if (MEAN) dq += dsv[i] * (mcol + cum[i]);
        if (GATE) {
          dq += dgv[i] * gwc;
          gsum += dgv[i] * (float)sQ[(tb + i) * LDK + col];
        }
        *pd_ = dq;
      }
    }
    if (GATE) {
      // column sums over the chunk's rows: one column's lanes across the four lane groups
      gsum += __shfl_xor(gsum, 16);
      gsum += __shfl_xor(gsum, 32);
      if (l < 16) sGp[col] = gsum;
    }
    if (MEAN) mcol += __shfl(cum[3], 48 + (l & 15));
#pragma unroll
    for (int ss = 0; ss < 2; ++ss)
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt) C[kt] = mfma16(frag16_tr(sK + 32 * ss * LDK + 16 * kt, LDK), kcol[ss], C[kt]);
    __syncthreads();

    // ---- 5: results of chunk c to registers (stored during the next pass); chunk c+1 in (each
    // thread overwrites exactly the sD pieces it read); k, q of chunk c+2
    out.read(sD, LDD, tid);
    sco = sScO[tid & (SB - 1)];
    dlo = sDlO[tid & (SB - 1)];
    if (GATE) {
      gpo = *(const f32x4*)(sGp + 4 * (tid % (K / 4)));
      dbo = sGp[K];
    }
    stage(min(c + 1, u.ce - 1));
    __syncthreads();
    load_a(min(c + 2, u.ce - 1));
  }
  put_out(u.ce - 1);
}

// ===========================================================================
// cs_gsum: grid N*H*nseg*NCB, CW/16 waves.  segG[:, cols] = sum over the segment of Q^T dZ[:, cols]
// (dZ = diag(f) dQc), segDM[cols] = sum of dm_t = -(s_t/pos_t) dz_t + ds_t q_t (every workgroup
// writes, zero when empty).  Reads the per-token scalars (f, ds, -s/pos) written by the dq walk
// (K <= 128) or by the per-token pass of the column walks (K = 256).  A workgroup loads q whole
// (the rows of G) and dQc only for its columns; the dm column sums are MFMAs of the per-token
// scalars (hi/lo, every output row the same) against the dZ and Q columns.
// ===========================================================================
template <int K, bool MEAN, bool DQ32>
__global__ __launch_bounds__(SegCols<K>::NT) void cs_gsum_kernel(const WalkArgs a) {
  constexpr int CW = SegCols<K>::CW, NT = SegCols<K>::NT, LDK = K + 16, LDZ = CW + 16, NKT = K / 16;
  constexpr int VPR = CW / 4;
  __shared__ __attribute__((aligned(16))) bf16 sQ[SB * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sZh[SB * LDZ];  // dZ[:, cols], hi
  __shared__ __attribute__((aligned(16))) bf16 sZl[SB * LDZ];
  // per token: ds, -s/pos as hi/lo bf16
  __shared__ __attribute__((aligned(16))) bf16 sDsH[SB], sDsL[SB], sSpH[SB], sSpL[SB];
  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(wave_id()), l = lane_id();
  const SegUnit u = seg_unit<K, SegCols<K>::NCB>(a);
  const int c0 = 16 * w, col = u.cbase + c0 + (l & 15), g4 = 4 * (l >> 4);
  auto chunk_len = [&](int c) { return min(SB, u.len - c * SB); };
  f32x4 G[NKT];
#pragma unroll
  for (int kt = 0; kt < NKT; ++kt) G[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 dm = f32x4{0.f, 0.f, 0.f, 0.f};
  RowsBf16<K, SB, NT> pq;
  RowsF32<CW, SB, NT> pd;
  constexpr int ND = RowsF32<CW, SB, NT>::N;
  f32x4 psc = f32x4{0.f, 0.f, 0.f, 0.f};  // per-token scalars of token (lane) of the chunk
  auto load = [&](int c) {
    const int L = chunk_len(c);
    const long off = u.hb + (long)c * SB * u.rs, tb = u.bos + (long)c * SB;
    pq.load((const bf16*)a.q + off, u.rs, L, tid);
    // (the upstream gradient's dtype is a template parameter: one load sequence)
    if (DQ32) pd.load(a.dqc32 + off + u.cbase, u.rs, L, tid);
    else pd.load(nullptr, (const bf16*)a.dqc16 + off + u.cbase, u.rs, L, tid);
    psc = *(const f32x4*)(a.sc + ((tb + min(tid & (SB - 1), L - 1)) * a.H + u.h) * 4);
  };
  auto stage = [&](int c) {
    const int L = chunk_len(c);
    pq.store(sQ, LDK, L, tid);
#pragma unroll
    for (int j = 0; j < ND; ++j) {
      const int idx = tid + j * NT, r = idx / VPR, cc = (idx % VPR) * 4;
      // f of row r from lane r (lane = token in psc)
      const float fr = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(4 * r, __builtin_bit_cast(int, psc[0])));
      const float f = r < L ? fr : 0.f;
      bf16x4 hh, ll;
      split4(f * pd.v[j], hh, ll);
      *(bf16x4*)(sZh + r * LDZ + cc) = hh;
      *(bf16x4*)(sZl + r * LDZ + cc) = ll;
    }
    if (MEAN && tid < SB) {
      const float ds = tid < L ? psc[1] : 0.f, sp = tid < L ? psc[3] : 0.f;
      bf16 x, y;
      split2(ds, x, y);
      sDsH[tid] = x;
      sDsL[tid] = y;
      split2(sp, x, y);
      sSpH[tid] = x;
      sSpL[tid] = y;
    }
  };
  // chunk loads and stages: unconditional (past the end the last chunk again)
  if (u.cb < u.ce) {
    load(u.cb);
    stage(u.cb);
    load(min(u.cb + 1, u.ce - 1));
  }
  __syncthreads();
  for (int c = u.cb; c < u.ce; ++c) {
#pragma unroll
    for (int ss = 0; ss < 2; ++ss) {
      const bf16x8 bh = frag16_tr(sZh + 32 * ss * LDZ + c0, LDZ), bl = frag16_tr(sZl + 32 * ss * LDZ + c0, LDZ);
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt) {
        const bf16x8 qa = frag16_tr(sQ + 32 * ss * LDK + 16 * kt, LDK);
        G[kt] = mfma16(qa, bh, G[kt]);
        G[kt] = mfma16(qa, bl, G[kt]);
      }
      if (MEAN) {
        // dm[cols] += sum_t (-s_t/pos_t) dz_t[cols] + ds_t q_t[cols]: A operands broadcast the
        // per-token scalars of slots t = 32 ss + 8 (lane / 16) + j to every row
        const int tb = 32 * ss + 8 * (l >> 4);
        const bf16x8 qc = frag16_tr(sQ + 32 * ss * LDK + u.cbase + c0, LDK);
        const bf16x8 ph = *(const bf16x8*)(sSpH + tb), pl = *(const bf16x8*)(sSpL + tb);
        const bf16x8 dh = *(const bf16x8*)(sDsH + tb), dl = *(const bf16x8*)(sDsL + tb);
        dm = mfma16(ph, bh, dm);
        dm = mfma16(ph, bl, dm);
        dm = mfma16(pl, bh, dm);
        dm = mfma16(dh, qc, dm);
        dm = mfma16(dl, qc, dm);
      }
    }
    __syncthreads();
    stage(min(c + 1, u.ce - 1));
    __syncthreads();
    load(min(c + 2, u.ce - 1));
  }
  float* dst = a.segG + ((long)u.unit * a.nseg + u.seg) * K * K;
#pragma unroll
  for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
    for (int r = 0; r < 4; ++r) dst[(long)(16 * kt + g4 + r) * K + col] = G[kt][r];
  // every row of the dm tile holds the column sums
  if (MEAN && l < 16) a.segDM[((long)u.unit * a.nseg + u.seg) * K + col] = dm[0];
}

// ===========================================================================
// cs_dk: grid N*H*nseg, K/16 waves, reverse walk of one segment.  State E[:, cols] (E = G + G^T +
// dC_T + dC_T^T over the chunks after the current one) and the dm carry start from the later
// segments' totals.  Per chunk (rows j, t of the chunk):
//   dK[:, cols] = K E[:, cols] + ((dZ K^T) o M)^T Q[:, cols] + ((Q K^T) o M)^T dZ[:, cols]
//                + sum_{t >= j} dm_t[cols] + carry[cols]     (+ dk_extra at the store)
//   E[:, cols] += Q^T dZ[:, cols] + dZ^T Q[:, cols];  carry += sum_t dm_t[cols]
// The dm suffix sums are two masked products: (t >= j ? ds_t : 0) against Q and (t >= j ?
// -s_t/pos_t : 0) against dZ.  Segment 0 also writes dC_0 = dC_T + sum_t q_t dz_t^T and dm_0.
// ===========================================================================
template <int K, bool MEAN, bool DQ32>
__global__ __launch_bounds__(K * 4) void cs_dk_kernel(const WalkArgs a) {
  static_assert(K <= 128, "segment walks hold all K columns of a (sequence, head) in one workgroup");
  constexpr int NW = K / 16, NT = 64 * NW;
  constexpr int LDK = K + 16, LDA = SB + 16, LDO = K + 4;
  constexpr int NKS = K / 32, NKT = K / 16, VPR = K / 4;
  __shared__ __attribute__((aligned(16))) bf16 sQ[SB * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sK[SB * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sZh[SB * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sZl[SB * LDK];
  // score planes: (Q K^T) o M hi, lo; (dZ K^T) o M hi, lo
  __shared__ __attribute__((aligned(16))) bf16 sAB[4 * SB * LDA];
  bf16* const sAh = sAB;
  bf16* const sAl = sAB + SB * LDA;
  bf16* const sBh = sAB + 2 * SB * LDA;
  bf16* const sBl = sAB + 3 * SB * LDA;
  __shared__ __attribute__((aligned(16))) float sO[SB * LDO];   // dk rows
  __shared__ __attribute__((aligned(16))) bf16 sDsH[SB], sDsL[SB], sSpH[SB], sSpL[SB];  // hi/lo of ds, -s/pos
  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(wave_id()), l = lane_id();
  const SegUnit u = seg_unit<K>(a);
  const bool first = u.seg == 0;
  if (u.cb >= u.ce && !first) return;
  const int c0 = 16 * w, col = c0 + (l & 15), g4 = 4 * (l >> 4);
  auto chunk_len = [&](int c) { return min(SB, u.len - c * SB); };

  // E at the end of the segment: later segments' G + G^T, plus dC_T + dC_T^T
  f32x4 E[NKT];
#pragma unroll
  for (int kt = 0; kt < NKT; ++kt) {
    E[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (a.dh_fin) {
      const float* p = a.dh_fin + (long)u.unit * K * K;
#pragma unroll
      for (int i = 0; i < 4; ++i) E[kt][i] = p[(long)(16 * kt + g4 + i) * K + col];
      E[kt] += *(const f32x4*)(p + (long)col * K + 16 * kt + g4);
    }
  }
  add_seg_tiles<K, true>(E, a.segG, u.unit, a.nseg, u.seg + 1, a.nseg, col, g4);
  float carry = 0.f;
  if (MEAN) {
    carry = a.dm_fin ? a.dm_fin[(long)u.unit * K + col] : 0.f;
    for (int s = u.seg + 1; s < a.nseg; ++s) carry += a.segDM[((long)u.unit * a.nseg + s) * K + col];
  }
#pragma unroll
  for (int kt = 0; kt < NKT; ++kt) settle(E[kt]);
  settle(carry);
  for (int i = tid; i < SB * LDA; i += NT) {
    sAh[i] = (bf16)0.f;
    sAl[i] = (bf16)0.f;
    sBh[i] = (bf16)0.f;
    sBl[i] = (bf16)0.f;
  }

  RowsBf16<K, SB, NT> pq, pk;
  RowsF32<K, SB, NT> pd;
  TileIn<K, NT> pe;  // dk_extra rows (zero when absent)
  constexpr int ND = RowsF32<K, SB, NT>::N;
  f32x4 psc = f32x4{0.f, 0.f, 0.f, 0.f};  // per-token scalars of token (lane) of the chunk
  // chunk loads in two parts, issued at different points of a pass so that the vector-memory
  // traffic of all workgroups spreads over the pass: k, q, the per-token scalars; the upstream
  // gradient and dk_extra
  auto load_a = [&](int c) {
    const int L = chunk_len(c);
    const long off = u.hb + (long)c * SB * u.rs, tb = u.bos + (long)c * SB;
    pk.load((const bf16*)a.k + off, u.rs, L, tid);
    pq.load((const bf16*)a.q + off, u.rs, L, tid);
    psc = *(const f32x4*)(a.sc + ((tb + min(tid & (SB - 1), L - 1)) * a.H + u.h) * 4);
  };
  auto load_b = [&](int c) {
    const int L = chunk_len(c);
    const long off = u.hb + (long)c * SB * u.rs;
    // (the upstream gradient's dtype is a template parameter: one load sequence)
    if (DQ32) pd.load(a.dqc32 + off, u.rs, L, tid);
    else pd.load(nullptr, (const bf16*)a.dqc16 + off, u.rs, L, tid);
    if (a.dk_extra) pe.load(rows_rsrc(a.dk_extra + off, u.rs, L, K, 4), u.rs, tid);
  };
  // chunk c into LDS; the dk rows start as dk_extra (each thread writes the sO pieces it stores)
  auto stage = [&](int c) {
    const int L = chunk_len(c);
    pk.store(sK, LDK, L, tid);
    pq.store(sQ, LDK, L, tid);
    if (a.dk_extra) pe.store(sO, LDO, tid);
    else TileIn<K, NT>{}.zero(sO, LDO, tid);
#pragma unroll
    for (int j = 0; j < ND; ++j) {
      const int idx = tid + j * NT, r = idx / VPR, cc = (idx % VPR) * 4;
      // f of row r from lane r (lane = token in psc)
      const float fr = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(4 * r, __builtin_bit_cast(int, psc[0])));
      const float f = r < L ? fr : 0.f;
      bf16x4 hh, ll;
      split4(f * pd.v[j], hh, ll);
      *(bf16x4*)(sZh + r * LDK + cc) = hh;
      *(bf16x4*)(sZl + r * LDK + cc) = ll;
    }
    if (tid < SB) {
      const float ds = tid < L ? psc[1] : 0.f, sp = tid < L ? psc[3] : 0.f;
      bf16 x, y;
      split2(ds, x, y);
      sDsH[tid] = x;
      sDsL[tid] = y;
      split2(sp, x, y);
      sSpH[tid] = x;
      sSpL[tid] = y;
    }
  };
  // mask of the suffix products' diagonal blocks: slot t = 8 (lane / 16) + j of row j' = lane % 16
  // (even row tiles) or 16 + lane % 16 (odd row tiles) is kept when t >= j' (formed where used: a
  // few compares are cheaper than eight registers held across the walk)
  auto diag_mask = [&](bool odd) {
    u32x4 m;
    const int j = (l & 15) + (odd ? 16 : 0);
#pragma unroll
    for (int wd = 0; wd < 4; ++wd) {
      const int t = 8 * (l >> 4) + 2 * wd;
      m[wd] = (t >= j ? 0x0000ffffu : 0u) | (t + 1 >= j ? 0xffff0000u : 0u);
    }
    return m;
  };
  // dk rows of a chunk, held in registers from the end of its pass to the next pass's stores
  TileOut<K, NT> out;
  auto put_out = [&](int pc) {
    const int L = chunk_len(pc);
    const long ob = u.hb + (long)pc * SB * u.rs;
    out.store(rows_rsrc(a.dk32 ? a.dk32 + ob : nullptr, u.rs, L, K, 4),
              rows_rsrc(a.dk ? (const bf16*)a.dk + ob : nullptr, u.rs, L, K, 2), u.rs, tid, a.dk32 != nullptr,
              a.dk != nullptr);
  };
  // chunk loads and stages: unconditional (past the start of the segment its first chunk again)
  if (u.cb < u.ce) {
    load_a(u.ce - 1);
    load_b(u.ce - 1);
    stage(u.ce - 1);
    load_a(max(u.ce - 2, u.cb));
  }
  __syncthreads();

  for (int c = u.ce - 1; c >= u.cb; --c) {
    const int L = chunk_len(c), t0 = c * SB;
    // ---- scores (e < 10: A = (Q K^T) o M, else B = (dZ K^T) o M)
#pragma unroll
    for (int j = 0; j < (20 + NW - 1) / NW; ++j) {
      const int e = w + j * NW;
      if (e < 20) {
        const int ee = e < 10 ? e : e - 10, I = tile_t(ee), J = tile_s(ee);
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
        if (e < 10) {
#pragma unroll
          for (int ks = 0; ks < NKS; ++ks)
            acc = mfma16(frag16_rm(sK + 16 * J * LDK + 32 * ks, LDK), frag16_rm(sQ + 16 * I * LDK + 32 * ks, LDK), acc);
        } else {
#pragma unroll
          for (int ks = 0; ks < NKS; ++ks) {
            const bf16x8 kf = frag16_rm(sK + 16 * J * LDK + 32 * ks, LDK);
            acc = mfma16(kf, frag16_rm(sZh + 16 * I * LDK + 32 * ks, LDK), acc);
            acc = mfma16(kf, frag16_rm(sZl + 16 * I * LDK + 32 * ks, LDK), acc);
          }
        }
        if (I == J) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (g4 + i > (l & 15)) acc[i] = 0.f;
        }
        score_to_lds(acc, sAB, SB * LDA, LDA, (e < 10 ? 0 : 2 * SB * LDA) + 16 * I * LDA + 16 * J);
      }
    }
    __syncthreads();
    // the previous (later) chunk's dk rows leave while this chunk's products run
    if (c < u.ce - 1) put_out(c + 1);

    // ---- dK rows, one 16-row tile (jt) at a time; the dm total of the chunk (row 0 of the suffix)
    bf16x8 qcol[2], zcolh[2], zcoll[2];
#pragma unroll
    for (int ts = 0; ts < 2; ++ts) {
      qcol[ts] = frag16_tr(sQ + 32 * ts * LDK + c0, LDK);
      zcolh[ts] = frag16_tr(sZh + 32 * ts * LDK + c0, LDK);
      zcoll[ts] = frag16_tr(sZl + 32 * ts * LDK + c0, LDK);
    }
    bf16x8 eh[NKS], el[NKS];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) acc_pair_split(E[2 * ks], E[2 * ks + 1], eh[ks], el[ks]);
    float dmtot = 0.f;
#pragma unroll 1
    for (int jt = 0; jt < 4; ++jt) {
      f32x4 xh = f32x4{0.f, 0.f, 0.f, 0.f}, xl = f32x4{0.f, 0.f, 0.f, 0.f}, sfx = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const bf16x8 ka = frag16_rm_acc(sK + 16 * jt * LDK + 32 * ks, LDK);
        xh = mfma16(ka, eh[ks], xh);
        xl = mfma16(ka, el[ks], xl);
      }
#pragma unroll
      for (int ts = 0; ts < 2; ++ts) {
        if (ts >= (jt >> 1)) {
          // B^T Q and A^T dZ: rows j of the transposed score tiles (transposing reads of [t][j])
          const bf16x8 bth = frag16_tr(sBh + 32 * ts * LDA + 16 * jt, LDA);
          const bf16x8 btl = frag16_tr(sBl + 32 * ts * LDA + 16 * jt, LDA);
          const bf16x8 ath = frag16_tr(sAh + 32 * ts * LDA + 16 * jt, LDA);
          const bf16x8 atl = frag16_tr(sAl + 32 * ts * LDA + 16 * jt, LDA);
          xh = mfma16(bth, qcol[ts], xh);
          xl = mfma16(btl, qcol[ts], xl);
          xh = mfma16(ath, zcolh[ts], xh);
          xl = mfma16(atl, zcolh[ts], xl);
          xl = mfma16(ath, zcoll[ts], xl);
          if (MEAN) {
            // masked diagonals: row j = 16 jt + (l & 15), slots t = 32 ts + 8 (l >> 4) + i, kept
            // for t >= j (whole step below the diagonal block, else the block's mask)
            const int tb = 32 * ts + 8 * (l >> 4);
            u32x4 m = u32x4{~0u, ~0u, ~0u, ~0u};
            if (ts == (jt >> 1)) m = diag_mask(jt & 1);
            const bf16x8 dh = __builtin_bit_cast(bf16x8, *(const u32x4*)(sDsH + tb) & m);
            const bf16x8 dl = __builtin_bit_cast(bf16x8, *(const u32x4*)(sDsL + tb) & m);
            const bf16x8 ph = __builtin_bit_cast(bf16x8, *(const u32x4*)(sSpH + tb) & m);
            const bf16x8 pl = __builtin_bit_cast(bf16x8, *(const u32x4*)(sSpL + tb) & m);
            sfx = mfma16(dh, qcol[ts], sfx);
            sfx = mfma16(dl, qcol[ts], sfx);
            sfx = mfma16(ph, zcolh[ts], sfx);
            sfx = mfma16(ph, zcoll[ts], sfx);
            sfx = mfma16(pl, zcolh[ts], sfx);
          }
        }
      }
      if (MEAN && jt == 0) dmtot = __shfl(sfx[0], l & 15);
#pragma unroll
      for (int i = 0; i < 4; ++i) sO[(16 * jt + g4 + i) * LDO + col] += xh[i] + xl[i] + sfx[i] + carry;
    }
    if (MEAN) carry += dmtot;
    // the upstream gradient and dk_extra of chunk c-1 (their registers were staged at the end of the
    // last pass)
    load_b(max(c - 1, u.cb));

    // ---- E[:, cols] += Q^T dZ[:, cols] + dZ^T Q[:, cols]
#pragma unroll
    for (int ts = 0; ts < 2; ++ts)
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt) {
        const bf16x8 qa = frag16_tr(sQ + 32 * ts * LDK + 16 * kt, LDK);
        const bf16x8 za = frag16_tr(sZh + 32 * ts * LDK + 16 * kt, LDK);
        const bf16x8 zb = frag16_tr(sZl + 32 * ts * LDK + 16 * kt, LDK);
        E[kt] = mfma16(qa, zcolh[ts], E[kt]);
        E[kt] = mfma16(qa, zcoll[ts], E[kt]);
        E[kt] = mfma16(za, qcol[ts], E[kt]);
        E[kt] = mfma16(zb, qcol[ts], E[kt]);
      }
    __syncthreads();
    // dk rows of chunk c to registers (stored during the next pass); chunk c-1 in; k, q of chunk c-2
    out.read(sO, LDO, tid);
    stage(max(c - 1, u.cb));
    __syncthreads();
    load_a(max(c - 2, u.cb));
  }
  if (u.cb < u.ce) put_out(u.cb);

  if (first) {
    if (a.dh0) {
      f32x4 D[NKT];
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          D[kt][i] = a.dh_fin ? a.dh_fin[((long)u.unit * K + 16 * kt + g4 + i) * K + col] : 0.f;
      }
      add_seg_tiles<K, false>(D, a.segG, u.unit, a.nseg, 0, a.nseg, col, g4);
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) a.dh0[((long)u.unit * K + 16 * kt + g4 + i) * K + col] = D[kt][i];
    }
    if (MEAN && a.dm0 && l < 16) a.dm0[(long)u.unit * K + col] = carry;
  }
}

// ===========================================================================
// launchers
// ===========================================================================
namespace {

int seg_cu_count() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cache[dev] <= 0) {
    int nn = 0;
    if (hipDeviceGetAttribute(&nn, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || nn <= 0) nn = 256;
    cache[dev] = nn;
  }
  return cache[dev];
}

// The segment sums (the sums and the gradient sums), SegCols<K>::NCB workgroups per (sequence, head,
// segment); for K = 256 the only segment kernels (its walks are column walks).
template <int K>
hipError_t cseg_sums_k(int stage, const WalkArgs& a, hipStream_t st) {
  const long wgs = (long)a.N * a.H * a.nseg * SegCols<K>::NCB;
  if (wgs <= 0) return hipSuccess;
  const dim3 grid((unsigned)wgs), block(SegCols<K>::NT);
  const bool mean = a.subtract_mean != 0;
  switch (stage) {
    case kSegSum:
      hipLaunchKernelGGL(cs_sum_kernel<K>, grid, block, 0, st, a);
      break;
    case kSegGsum:
      if (a.dqc32) {
        if (mean) hipLaunchKernelGGL((cs_gsum_kernel<K, true, true>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((cs_gsum_kernel<K, false, true>), grid, block, 0, st, a);
      } else {
        if (mean) hipLaunchKernelGGL((cs_gsum_kernel<K, true, false>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((cs_gsum_kernel<K, false, false>), grid, block, 0, st, a);
      }
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int K>
hipError_t cseg_k(int stage, const WalkArgs& a, hipStream_t st) {
  if (stage == kSegSum || stage == kSegGsum) return cseg_sums_k<K>(stage, a, st);
  const long wgs = (long)a.N * a.H * a.nseg;
  if (wgs <= 0) return hipSuccess;
  const dim3 grid((unsigned)wgs), block(K * 4);
  const bool mean = a.subtract_mean != 0, gate = a.gate_w != nullptr;
  switch (stage) {
    case kSegFwd:
      if (mean && gate) hipLaunchKernelGGL((cs_fwd_kernel<K, true, true>), grid, block, 0, st, a);
      else if (mean) hipLaunchKernelGGL((cs_fwd_kernel<K, true, false>), grid, block, 0, st, a);
      else if (gate) hipLaunchKernelGGL((cs_fwd_kernel<K, false, true>), grid, block, 0, st, a);
      else hipLaunchKernelGGL((cs_fwd_kernel<K, false, false>), grid, block, 0, st, a);
      break;
    case kSegDq: {
      const int sel = (a.dqc32 ? 4 : 0) + (mean ? 2 : 0) + (gate ? 1 : 0);
#define CCQ_SEG_DQ(S, A, B, C) \
  case S: hipLaunchKernelGGL((cs_dq_kernel<K, B, C, A>), grid, block, 0, st, a); break;
      switch (sel) {
        CCQ_SEG_DQ(0, false, false, false) CCQ_SEG_DQ(1, false, false, true) CCQ_SEG_DQ(2, false, true, false)
        CCQ_SEG_DQ(3, false, true, true) CCQ_SEG_DQ(4, true, false, false) CCQ_SEG_DQ(5, true, false, true)
        CCQ_SEG_DQ(6, true, true, false) CCQ_SEG_DQ(7, true, true, true)
      }
#undef CCQ_SEG_DQ
      break;
    }
    case kSegDk:
      if (a.dqc32) {
        if (mean) hipLaunchKernelGGL((cs_dk_kernel<K, true, true>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((cs_dk_kernel<K, false, true>), grid, block, 0, st, a);
      } else {
        if (mean) hipLaunchKernelGGL((cs_dk_kernel<K, true, false>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((cs_dk_kernel<K, false, false>), grid, block, 0, st, a);
      }
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

// Segments per sequence, at least two 64-token chunks each (T: the dense length, or the packed
// length of a varlen batch).  Segment walks (K in {64, 128}): enough workgroups to cover the CUs.
// K = 256: its column walks run K / 32 workgroups per (sequence, head) and segment, one per CU:
// as many segments as fill the CUs without a second round of workgroups.
int cseg_count(int N, int H, int T, int K) {
  const long units = (long)N * H;
  if (units <= 0) return 1;
  const int chunks = (T + SB - 1) / SB;
  int nseg;
  if (K > 128) nseg = (int)(seg_cu_count() / (units * (K / 32)));
  else nseg = (int)((seg_cu_count() + units - 1) / units);
  nseg = min(nseg, max(1, chunks / 2));
  return max(1, min(nseg, 16));
}

bool cseg_supported(int K) { return K == 64 || K == 128; }
bool cseg_sums_supported(int K) { return K == 64 || K == 128 || K == 256; }

hipError_t launch_cseg(int stage, const WalkArgs& a, hipStream_t st) {
  switch (a.K) {
    case 64: return cseg_k<64>(stage, a, st);
    case 128: return cseg_k<128>(stage, a, st);
    case 256: return cseg_sums_k<256>(stage, a, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ccq
