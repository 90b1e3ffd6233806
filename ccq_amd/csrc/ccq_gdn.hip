// Gated delta rule, chunked (chunk size 64), forward and backward, on gfx950.
//
// Recurrence (arXiv:2412.06464; the backbone the reference calls through
// fla's chunk_gated_delta_rule, ccq/ops/ccq_gdn/fused_chunk.py:54-58):
//   S <- exp(g_t) S;  u_t = beta_t (v_t - S^T k_t);  S <- S + k_t u_t^T;  o_t = S^T (scale q_t)
// Per chunk, with G the in-chunk cumulative sum of g, gamma = exp(G),
// Gamma_ij = exp(G_i - G_j), L1 = last row:
//   A = strict_lower(diag(beta) (K K^T o Gamma)),  T = (I + A)^-1
//   w = T diag(beta gamma) K,  u = T diag(beta) V,  U = u - w S
//   O = scale diag(gamma) Q S + P U,  P = scale (Q K^T o Gamma), causal incl. diagonal
//   S <- gamma_L S + K^T diag(gamma_L / gamma) U
//
// Kernels:
//   gdn_prep         chunk-parallel: G, T, w, u
//   gdn_fwd_state    one workgroup per (sequence, head, 32 state columns), walks the chunks:
//                    U, state snapshots hT
//   gdn_fwd_o        chunk-parallel: P (kept for the backward as P^T) and O
//   gdn_bwd_state    reverse walk per (sequence, head, 32 state columns): dU, dS snapshots dhT
//   gdn_bwd_dqkw     chunk x 64-column tiles of K: dq, the state/output part of dk, dw, dG partials
//   gdn_bwd_wy       chunk-parallel: backward through the WY representation -> dk, dv, dbeta, dg
//
// Precision: products whose operands are the bf16 inputs run as one bf16 MFMA; the
// operands that carry the leading part of a result (U, P, the cleaned query, dU, ...)
// are fed as hi/lo bf16 pairs so every result keeps ~16 significant bits.
#include "ccq_tile.h"
#include "ccq_params.h"

#include <type_traits>

namespace ccq {

namespace {

constexpr int BT = 64;

// Offset (in rows) of accumulator element i from the lane's first row (acc_row(0)).
__device__ __forceinline__ constexpr int acc_drow(int i) { return 8 * (i >> 2) + (i & 3); }

// Lower 32 x 32 block b of a 64 x 64 tile (row block, column block): 0 -> (0,0), 1 -> (1,0), 2 -> (1,1).
__device__ __forceinline__ int blk_row3(int b) { return b == 0 ? 0 : 1; }
__device__ __forceinline__ int blk_col3(int b) { return b == 2 ? 1 : 0; }

struct Carver {
  char* p;
  template <typename T>
  __device__ __forceinline__ T* take(int n) {
    T* r = (T*)p;
    p += ((long)n * sizeof(T) + 15) & ~15L;
    return r;
  }
};

// Returns false for the padding entries of a varlen launch (grid sized by an upper bound).
__device__ __forceinline__ bool chunk_info(const GdnArgs& a, int gc, int& n, int& c0, long& bos, int& L) {
  if (a.cu) {
    n = a.chunk_idx[2 * gc];
    if (n < 0) return false;
    const int c = a.chunk_idx[2 * gc + 1];
    bos = (long)a.cu[n];
    const int len = (int)(a.cu[n + 1] - a.cu[n]);
    c0 = c * BT;
    L = min(BT, len - c0);
  } else {
    n = gc / a.NT;
    const int c = gc % a.NT;
    bos = (long)n * a.T;
    c0 = c * BT;
    L = min(BT, a.T - c0);
  }
  return true;
}

// Rows of fp32 or bf16 into fp32 LDS (row-major and/or transposed), zero-filled past nvalid.
template <int D>
__device__ __forceinline__ void stage_any_f32(float* dst, int ld, float* dst_t, int ldt, const float* g32,
                                              const bf16* g16, long gstride, int rows, int nvalid) {
  if (g32) {
    stage_f32<D>(dst, ld, dst_t, ldt, g32, gstride, rows, nvalid);
    return;
  }
  constexpr int VPR = D / 8;
  for (int idx = threadIdx.x; idx < rows * VPR; idx += kThreads) {
    const int r = idx / VPR, c = (idx % VPR) * 8;
    bf16x8 v;
    if (r < nvalid) {
      v = *(const bf16x8*)(g16 + (long)r * gstride + c);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = (bf16)0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (dst) dst[r * ld + c + i] = (float)v[i];
      if (dst_t) dst_t[(c + i) * ldt + r] = (float)v[i];
    }
  }
}

// Copy `rows` rows of D bf16 from LDS (leading dim ld) to global (row stride gstride), 16-byte vectors.
template <int D>
__device__ __forceinline__ void lds_to_global_bf16(bf16* g, long gstride, const bf16* s, int ld, int rows) {
  constexpr int VPR = D / 8;
  for (int idx = threadIdx.x; idx < rows * VPR; idx += kThreads) {
    const int r = idx / VPR, c = (idx % VPR) * 8;
    *(bf16x8*)(g + (long)r * gstride + c) = *(const bf16x8*)(s + r * ld + c);
  }
}

// ===========================================================================
// Snapshot rows in block floating point: 16-bit integers with a power-of-two scale per row.  A
// [rows][K] snapshot held in LDS as hi/lo bf16 pairs leaves as round(x / 2^e_r) in int16 and 2^e_r in
// fp32, e_r = floor(log2 max_k |x|) - 14: the row's largest element keeps 15 significant bits and
// every element an absolute error of at most 2^-16 of it -- about the hi/lo pair's precision on the
// dense rows of a state, in half its bytes (an fp16 row keeps 11 bits per element, which the dk of
// the backward measurably felt).  The scale stays a normal fp32 number (e_r >= -126): a row whose
// largest element is below 2^-112 keeps an absolute error below 2^-127.  The K / 8 consecutive lanes
// that hold a row (8 elements each) find its largest magnitude by DPP lane moves within the wave's
// 16-lane rows, so no barrier and no LDS round trip is needed; every lane of the wave takes part.
// A consumer multiplies the integer back by the exact power-of-two scale in fp32 and splits the
// value into its usual hi/lo pair.
// ===========================================================================
typedef short i16x8 __attribute__((ext_vector_type(8)));

// Maximum of v over each aligned group of G consecutive lanes (G a power of two, 2..64): quad
// permutations for lanes 1 and 2 apart, the half-row and row mirrors for 4 and 8 apart (after the
// steps before them every lane of a quad, then of a half-row, holds the same value), a lane swap
// beyond 16.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// The magnitudes are taken as bit patterns (sign bit cleared): for non-negative floats the unsigned
// order of the patterns is the numeric order, so the maxima are integer maxima, whose lane moves fold
// into the max as DPP operands (a float max canonicalises both operands first).  Beyond 16 lanes the
// permlane swaps leave each lane's own value in one result and its partner's in the other.
template <int CTRL>
__device__ __forceinline__ unsigned umax_dpp(unsigned x) {
  return max(x, (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xf, 0xf, false));
}

template <int G>
__device__ __forceinline__ unsigned group_umax(unsigned v) {
  if constexpr (G >= 2) v = umax_dpp<0xB1>(v);    // quad_perm [1, 0, 3, 2]
  if constexpr (G >= 4) v = umax_dpp<0x4E>(v);    // quad_perm [2, 3, 0, 1]
  if constexpr (G >= 8) v = umax_dpp<0x141>(v);   // row_half_mirror
  if constexpr (G >= 16) v = umax_dpp<0x140>(v);  // row_mirror
  if constexpr (G >= 32) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = max((unsigned)r[0], (unsigned)r[1]);
  }
  if constexpr (G >= 64) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    v = max((unsigned)r[0], (unsigned)r[1]);
  }
  return v;
}

template <int K>
__device__ __forceinline__ void snap16_store(const bf16* hi, const bf16* lo, short* dst, float* dst_scale, int lane) {
  constexpr int G = K / 8;  // lanes per row
  float x[8];
  unsigned mx = 0;  // bit pattern of the largest |x|
  const bf16x8 h8 = *(const bf16x8*)hi, l8 = *(const bf16x8*)lo;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    x[i] = (float)h8[i] + (float)l8[i];
    mx = max(mx, __float_as_uint(x[i]) & 0x7fffffffu);
  }
  mx = group_umax<G>(mx);
  // floor(log2 mx) from the exponent field (0 and subnormal maxima land on the lower clamp)
  const int e = min(max((int)((mx >> 23) & 0xff) - 127 - 14, -126), 113);
  i16x8 out;
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = (short)__builtin_amdgcn_fmed3f(rintf(ldexpf(x[i], -e)), -32767.f, 32767.f);
  *gmem((i16x8*)dst) = out;
  if ((lane & (G - 1)) == 0) *gmem(dst_scale) = ldexpf(1.f, e);
}

}  // namespace

// ===========================================================================
// gdn_prep: grid (NTG, H)
// ===========================================================================
template <int K>
__global__ __launch_bounds__(kThreads) void gdn_prep_kernel(const GdnArgs a, const int V) {
  constexpr int LDK = K + 8, LDB = BT + 8, LDT = BT + 1;
  constexpr long kBytes = (long)BT * LDK * 2 + (long)K * LDB * 2 + 2L * BT * LDT * 4 + 4 * 256 * 4 + 3 * 256 * 4 +
                          4 * BT * 4 + 16 * 12;
  __shared__ __attribute__((aligned(16))) char smem[kBytes];
  Carver cv{smem};
  bf16* sK = cv.take<bf16>(BT * LDK);
  bf16* sKT = cv.take<bf16>(K * LDB);
  float* sA = cv.take<float>(BT * LDT);   // A, later T
  float* sTo = cv.take<float>(BT * LDT);  // off-diagonal blocks of T
  bf16* sVT = sK;                         // value tiles reuse the K rows once A is formed
  float* sD = cv.take<float>(4 * 256);    // inverses of the 16x16 diagonal blocks
  float* sScr = cv.take<float>(3 * 256);
  float* sG = cv.take<float>(BT);
  float* sBeta = cv.take<float>(BT);
  float* sGam = cv.take<float>(BT);
  float* sBG = cv.take<float>(BT);  // beta * gamma

  const int tid = threadIdx.x, w = wave_id(), l = lane_id();
  const int gc = blockIdx.x, h = blockIdx.y;
  int n, c0, L;
  long bos;
  if (!chunk_info(a, gc, n, c0, bos, L)) return;
  const long tok0 = bos + c0;
  const long rsk = (long)a.H * K, rsv = (long)a.H * V;

  // value tiles, one 64-column block ahead (the first one loads with K)
  const bf16* vg = (const bf16*)a.v + (tok0 * a.H + h) * (long)V;
  PrefetchBf16<64, BT> pV;
  pV.load(vg, rsv, L);
  stage_bf16<K>(sK, LDK, sKT, LDB, (const bf16*)a.k + (tok0 * a.H + h) * K, rsk, BT, L);
  if (w == 0) {
    float x = (l < L && a.g) ? a.g[(tok0 + l) * a.H + h] : 0.f;
    x = wave_scan_incl(x);
    sG[l] = x;
    sBeta[l] = (l < L) ? a.beta[(tok0 + l) * a.H + h] : 0.f;
    sGam[l] = __expf(x);
    sBG[l] = sBeta[l] * sGam[l];
    if (l < L) a.gcum[(tok0 + l) * a.H + h] = x;
  }
  __syncthreads();

  // A = strict_lower(beta_i Gamma_ij (K K^T)_ij)
  if (w < 3) {
    const int tr = (w == 0) ? 0 : 1, tc = (w == 2) ? 1 : 0;
    f32x16 acc = zero16();
    mma_rr(acc, sK + tr * 32 * LDK, LDK, sK + tc * 32 * LDK, LDK, K);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = tr * 32 + acc_row(i), c = tc * 32 + acc_col();
      sA[r * LDT + c] = (r > c) ? sBeta[r] * __expf(sG[r] - sG[c]) * acc[i] : 0.f;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) sA[acc_row(i) * LDT + 32 + acc_col()] = 0.f;
  }
  __syncthreads();

  // T = (I + A)^-1 by 16x16 blocks: diagonal blocks by forward substitution ...
  if (tid < 64) {
    const int b0 = (tid >> 4) * 16, col = tid & 15;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float s = (i == col) ? 1.f : 0.f;
#pragma unroll
      for (int m = 0; m < i; ++m) s -= sA[(b0 + i) * LDT + b0 + m] * x[m];
      x[i] = s;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sD[(tid >> 4) * 256 + i * 16 + col] = x[i];
  }
  __syncthreads();
  // ... then off-diagonal blocks by distance d:  T_IJ = -T_II sum_{M=J}^{I-1} A_IM T_MJ
  for (int d = 1; d < 4; ++d) {
    const int np = 4 - d;
    for (int e = tid; e < np * 256; e += kThreads) {
      const int p = e >> 8, r = (e >> 4) & 15, c = e & 15;
      const int I = p + d, J = p;
      float s = 0.f;
      for (int M = J; M < I; ++M) {
        for (int m = 0; m < 16; ++m) {
          const float tmj = (M == J) ? sD[J * 256 + m * 16 + c] : sTo[(M * 16 + m) * LDT + J * 16 + c];
          s += sA[(I * 16 + r) * LDT + M * 16 + m] * tmj;
        }
      }
      sScr[p * 256 + r * 16 + c] = s;
    }
    __syncthreads();
    for (int e = tid; e < np * 256; e += kThreads) {
      const int p = e >> 8, r = (e >> 4) & 15, c = e & 15;
      const int I = p + d, J = p;
      float s = 0.f;
      for (int m = 0; m < 16; ++m) s += sD[I * 256 + r * 16 + m] * sScr[p * 256 + m * 16 + c];
      sTo[(I * 16 + r) * LDT + J * 16 + c] = -s;
    }
    __syncthreads();
  }
  // assemble T into sA and the fp32 copy for the backward
  float* tg = a.tmat + ((long)gc * a.H + h) * (BT * BT);
  for (int e = tid; e < BT * BT; e += kThreads) {
    const int r = e >> 6, c = e & 63;
    const int I = r >> 4, J = c >> 4;
    float t;
    if (I == J) t = sD[I * 256 + (r & 15) * 16 + (c & 15)];
    else if (I > J) t = sTo[r * LDT + c];
    else t = 0.f;
    sA[r * LDT + c] = t;
    tg[e] = t;
  }
  __syncthreads();

  // w = (T diag(beta gamma)) K  (64 x K); the column scaling is applied in fp32 and the
  // scaled T enters as a hi/lo pair (beta itself is not a bf16 number in general)
  {
    bf16* wg = (bf16*)a.w + (tok0 * a.H + h) * K;
    bf16* wlg = (bf16*)a.wl + (tok0 * a.H + h) * K;
    for (int tile = w; tile < 2 * (K / 32); tile += 4) {
      const int tr = tile & 1, tc = tile >> 1;
      f32x16 acc = zero16();
      for (int k0 = 0; k0 < BT; k0 += 16) {
        bf16x8 hi, lo;
        frag_rm_f32_ks(sA + tr * 32 * LDT + k0, LDT, sBG + k0, hi, lo);
        const bf16x8 b = frag_rm(sKT + tc * 32 * LDB + k0, LDB);
        acc = mfma(hi, b, acc);
        acc = mfma(lo, b, acc);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = tr * 32 + acc_row(i);
        if (r < L) {
          bf16 hi, lo;
          split2(acc[i], hi, lo);
          wg[(long)r * rsk + tc * 32 + acc_col()] = hi;
          wlg[(long)r * rsk + tc * 32 + acc_col()] = lo;
        }
      }
    }
  }
  // u = (T diag(beta)) V  (64 x V), 64 value columns at a time
  float* ug = a.u + (tok0 * a.H + h) * (long)V;
  for (int v0 = 0; v0 < V; v0 += 64) {
    pV.store(nullptr, 0, sVT, LDB);
    __syncthreads();
    if (v0 + 64 < V) pV.load(vg + v0 + 64, rsv, L);
    {
      const int tr = w & 1, tc = w >> 1;
      f32x16 acc = zero16();
      for (int k0 = 0; k0 < BT; k0 += 16) {
        bf16x8 hi, lo;
        frag_rm_f32_ks(sA + tr * 32 * LDT + k0, LDT, sBeta + k0, hi, lo);
        const bf16x8 b = frag_rm(sVT + tc * 32 * LDB + k0, LDB);
        acc = mfma(hi, b, acc);
        acc = mfma(lo, b, acc);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = tr * 32 + acc_row(i);
        if (r < L) ug[(long)r * rsv + v0 + tc * 32 + acc_col()] = acc[i];
      }
    }
    __syncthreads();
  }
}

// ===========================================================================
// gdn_prep for K, V in {64, 128}: persistent workgroups of 8 waves, one per CU, over the (chunk,
// head) units.  Waves 4-7 load the next unit's k, v, g and beta into registers while waves 0-3 work,
// and write them into LDS (with the in-chunk cumulative g, which they also store) once the current
// unit is done.  Per unit, on waves 0-3:
//   P1  A = strict_lower(beta_r Gamma_rc (K K^T)_rc) (three 32x32 MFMA blocks), fp32 in LDS
//   P2  the four 16x16 diagonal blocks D_I = (I + A_II)^-1 by forward substitution (fp32, one
//       column per lane)
//   P3  the 32-level blocks T_{2p+1,2p} = -D_{2p+1} A_{2p+1,2p} D_{2p} (fp32 on the VALU)
//   P4  the 64-level block T_10 = -T_1 (A_10 T_0) (32x32 MFMA products on hi/lo operands)
//   P5  T diag(beta gamma) and T diag(beta) as hi/lo row tiles; T (fp32, hi + lo) to HBM
//   P6  w^T = K^T (T diag(beta gamma))^T and u^T = V^T (T diag(beta))^T tiles, staged per wave in
//       the A / T buffers and stored as whole rows (w as its hi/lo pair); rows past the chunk are
//       dropped by range-checked buffer stores
// T is unit lower triangular; its upper blocks are zeroed once and never written.
// ===========================================================================
template <int K, int V>
__global__ __launch_bounds__(kWalk8) void gdn_prep_v3_kernel(const GdnArgs a) {
  constexpr int PT = BT + 8, PF = BT + 4, PK = K + 8, PV = V + 8, PX = 32 + 40, NM = 256;
  constexpr int NKB = K / 32, NVB = V / 32, NJK = NKB / 2, NJV = NVB / 2;
  static_assert(NKB % 2 == 0 && NVB % 2 == 0, "two column groups of tiles");
  __shared__ __attribute__((aligned(16))) bf16 sK[BT * PK];                 // k [t][k]
  __shared__ __attribute__((aligned(16))) bf16 sV[BT * PV];                 // v [t][v]
  __shared__ __attribute__((aligned(16))) float sA[BT * PF];                // A [r][c]
  __shared__ __attribute__((aligned(16))) float sTf[BT * PF];               // T, blocks formed on the VALU
  __shared__ __attribute__((aligned(16))) bf16 sTh[BT * PT], sTl[BT * PT];  // T [r][c]
  __shared__ __attribute__((aligned(16))) bf16 sXh[32 * PX], sXl[32 * PX];  // X = A_10 T_0 [r][c]
  __shared__ __attribute__((aligned(16))) bf16 sBh[BT * PT], sBl[BT * PT];  // T diag(beta gamma) [t][s]
  __shared__ __attribute__((aligned(16))) bf16 sCh[BT * PT], sCl[BT * PT];  // T diag(beta) [t][s]
  __shared__ __attribute__((aligned(16))) float sG[BT], sBeta[BT], sBG[BT];
  __shared__ __attribute__((aligned(16))) float sY[2 * 256];                // A_{2p+1,2p} D_{2p}

  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(wave_id()), l = lane_id();
  const int nunits = a.NTG * a.H;
  const long rsk = (long)a.H * K, rsv = (long)a.H * V;
  auto valid_from = [&](int u) {
    for (; u < nunits; u += gridDim.x) {
      int n, c0, L;
      long bos;
      if (chunk_info(a, u / a.H, n, c0, bos, L)) break;
    }
    return u;
  };

  if (w >= 4) {
    // ---------------- memory waves
    const int lm = tid - NM;
    RowsBf16<K, BT, NM> pk;
    RowsBf16<V, BT, NM> pv;
    float pg = 0.f, pb = 0.f;  // raw g and beta of token l (consumed at staging)
    int L = 0, h = 0;
    long tok0 = 0;
    auto locate = [&](int u) {
      h = u % a.H;
      int n, c0;
      long bos;
      chunk_info(a, u / a.H, n, c0, bos, L);
      tok0 = bos + c0;
    };
    auto load = [&]() {
      pk.load((const bf16*)a.k + (tok0 * a.H + h) * K, rsk, L, lm);
      pv.load((const bf16*)a.v + (tok0 * a.H + h) * (long)V, rsv, L, lm);
      const long tk = (tok0 + min(l, L - 1)) * a.H + h;
      pg = a.g ? *gmem(a.g + tk) : 0.f;
      pb = *gmem(a.beta + tk);
    };
    // k, v rows (zero past the chunk); wave 4: in-chunk inclusive cumsum of g (the last token's
    // beyond the chunk), beta (0 beyond it), beta gamma, and the cumulative g to HBM
    auto stage = [&]() {
      pk.store(sK, PK, L, lm);
      pv.store(sV, PV, L, lm);
      if (w == 4) {
        float x = l < L ? pg : 0.f;
        x = wave_scan_incl(x);
        const float b = l < L ? pb : 0.f;
        sG[l] = x;
        sBeta[l] = b;
        sBG[l] = b * __expf(x);
        if (l < L) a.gcum[(tok0 + l) * a.H + h] = x;
      }
    };
    int u = valid_from(blockIdx.x);
    if (u < nunits) {
      locate(u);
      load();
      stage();
    }
    int un = u < nunits ? valid_from(u + gridDim.x) : nunits;
    while (u < nunits) {
      const bool more = un < nunits;
      if (more) locate(un);
      __syncthreads();  // B0
      if (more) load();
      __syncthreads();  // B1
      __syncthreads();  // B2
      __syncthreads();  // B3
      __syncthreads();  // B4
      __syncthreads();  // B5
      __syncthreads();  // B6
      __syncthreads();  // B7
      if (more) stage();
      u = un;
      un = u < nunits ? valid_from(u + gridDim.x) : nunits;
    }
    return;
  }

  // ---------------- compute waves
  // T's upper blocks (16x16 blocks (0,1), (2,3) and the 32x32 block (0,1)) stay zero
  for (int e = tid; e < BT * BT; e += NM) {
    const int r = e >> 6, c = e & 63;
    sTh[r * PT + c] = (bf16)0.f;
    sTl[r * PT + c] = (bf16)0.f;
  }
  const int R = blk_row3(w), C = blk_col3(w);
  const int tr = w >> 1;
  const int q4 = 4 * (l >> 5);
  const int ct = tid;  // 0..255
  for (int u = valid_from(blockIdx.x); u < nunits; u = valid_from(u + gridDim.x)) {
    const int gc = u / a.H, h = u % a.H;
    int n, c0, L;
    long bos;
    chunk_info(a, gc, n, c0, bos, L);
    const long tok0 = bos + c0;
    __syncthreads();  // B0: k, v, g, beta of the unit are in LDS

    // ---- P1: A (rows r, cols c) for the lower 32x32 blocks
    if (w < 3) {
      f32x16 acc = zero16(), acc2 = zero16();
#pragma unroll
      for (int k0 = 0; k0 < K; k0 += 32) {
        acc = mfma(frag_rm(sK + R * 32 * PK + k0, PK), frag_rm(sK + C * 32 * PK + k0, PK), acc);
        acc2 = mfma(frag_rm(sK + R * 32 * PK + k0 + 16, PK), frag_rm(sK + C * 32 * PK + k0 + 16, PK), acc2);
      }
      const int c = C * 32 + acc_col();
      const float gc_ = sG[c];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r0 = R * 32 + 8 * q + q4;
        const f32x4 grv = *(const f32x4*)(sG + r0), brv = *(const f32x4*)(sBeta + r0);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const bool keep = r0 + ii > c;
          const float e = __expf(keep ? grv[ii] - gc_ : 0.f);
          sA[(r0 + ii) * PF + c] = keep ? brv[ii] * e * (acc[4 * q + ii] + acc2[4 * q + ii]) : 0.f;
        }
      }
    }
    __syncthreads();  // B1

    // ---- P2: D_I = (I + A_II)^-1, block I = w, column l (lanes 0..15)
    if (l < 16) {
      const int b0 = 16 * w;
      float x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float s = (i == l) ? 1.f : 0.f;
#pragma unroll
        for (int m = 0; m < i; ++m) s -= sA[(b0 + i) * PF + b0 + m] * x[m];
        x[i] = s;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        sTf[(b0 + i) * PF + b0 + l] = x[i];
        bf16 hi, lo;
        split2(x[i], hi, lo);
        sTh[(b0 + i) * PT + b0 + l] = hi;
        sTl[(b0 + i) * PT + b0 + l] = lo;
      }
    }
    __syncthreads();  // B2

    // ---- P3: Y_p = A_{2p+1,2p} D_{2p};  T_{2p+1,2p} = -D_{2p+1} Y_p   (p = 0, 1; 16x16 each)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int e = ct + 256 * j, p = e >> 8, r = (e >> 4) & 15, c = e & 15;
      const float* ar = sA + (32 * p + 16 + r) * PF + 32 * p;
      const float* dc = sTf + (32 * p) * PF + 32 * p + c;
      float s = 0.f;
#pragma unroll
      for (int m = 0; m < 16; m += 4) {
        const f32x4 av = *(const f32x4*)(ar + m);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) s += av[ii] * dc[(m + ii) * PF];
      }
      sY[e] = s;
    }
    __syncthreads();  // B3
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int e = ct + 256 * j, p = e >> 8, r = (e >> 4) & 15, c = e & 15;
      const float* dr = sTf + (32 * p + 16 + r) * PF + 32 * p + 16;
      const float* yc = sY + p * 256 + c;
      float s = 0.f;
#pragma unroll
      for (int m = 0; m < 16; m += 4) {
        const f32x4 dv = *(const f32x4*)(dr + m);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) s += dv[ii] * yc[(m + ii) * 16];
      }
      const int row = 32 * p + 16 + r, col = 32 * p + c;
      bf16 hi, lo;
      split2(-s, hi, lo);
      sTh[row * PT + col] = hi;
      sTl[row * PT + col] = lo;
    }
    __syncthreads();  // B4

    // ---- P4 (wave 0): X^T = (A_10 T_0)^T (rows c, cols r), then T_10^T = -(T_1 X)^T
    if (w == 0) {
      f32x16 xt = zero16();
#pragma unroll
      for (int m0 = 0; m0 < 32; m0 += 16) {
        const bf16x8 th = frag32_tr(sTh + m0 * PT, PT), tl = frag32_tr(sTl + m0 * PT, PT);
        bf16x8 ah, al;
        frag_rm_f32(sA + 32 * PF + m0, PF, ah, al);
        xt = mfma(th, ah, xt);
        xt = mfma(th, al, xt);
        xt = mfma(tl, ah, xt);
      }
      acc_to_lds_t(xt, sXh, sXl, PX, 0);  // X [r][c]
      f32x16 tt = zero16();
#pragma unroll
      for (int m0 = 0; m0 < 32; m0 += 16) {
        const bf16x8 xh = frag32_tr(sXh + m0 * PX, PX), xl = frag32_tr(sXl + m0 * PX, PX);
        const bf16x8 bh = frag_rm(sTh + 32 * PT + 32 + m0, PT), bl = frag_rm(sTl + 32 * PT + 32 + m0, PT);
        tt = mfma(xh, bh, tt);
        tt = mfma(xh, bl, tt);
        tt = mfma(xl, bh, tt);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) tt[i] = -tt[i];
      acc_to_lds_t(tt, sTh + 32 * PT, sTl + 32 * PT, PT, 0);  // T[32 + r][c]
    }
    __syncthreads();  // B5

    // ---- P5: T diag(beta gamma), T diag(beta) (hi/lo rows) and T (fp32) to HBM; thread: rows
    // (ct >> 4) + 16 q, columns 4 (ct & 15) .. +3 (each row of T leaves as one 256-byte line)
    {
      const int c = 4 * (ct & 15);
      float* tg = a.tmat + ((long)gc * a.H + h) * (BT * BT) + c;
      const f32x4 bg = *(const f32x4*)(sBG + c), bt = *(const f32x4*)(sBeta + c);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int t = (ct >> 4) + 16 * q;
        const bf16x4 th = *(const bf16x4*)(sTh + t * PT + c), tl = *(const bf16x4*)(sTl + t * PT + c);
        f32x4 x;
        bf16x4 bh, bl, ch, cl;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x[i] = (float)th[i] + (float)tl[i];
          bf16 p, r;
          split2(x[i] * bg[i], p, r);
          bh[i] = p;
          bl[i] = r;
          split2(x[i] * bt[i], p, r);
          ch[i] = p;
          cl[i] = r;
        }
        *gmem((f32x4*)(tg + t * BT)) = x;
        *(bf16x4*)(sBh + t * PT + c) = bh;
        *(bf16x4*)(sBl + t * PT + c) = bl;
        *(bf16x4*)(sCh + t * PT + c) = ch;
        *(bf16x4*)(sCl + t * PT + c) = cl;
      }
    }
    __syncthreads();  // B6

    // ---- P6: w^T tiles (rows k, cols t) and u^T tiles (rows v, cols t)
    {
      const __amdgpu_buffer_rsrc_t rw = buf_rsrc((const bf16*)a.w + (tok0 * a.H + h) * K, (int)(((L - 1) * rsk + K) * 2));
      const __amdgpu_buffer_rsrc_t rwl = buf_rsrc((const bf16*)a.wl + (tok0 * a.H + h) * K, (int)(((L - 1) * rsk + K) * 2));
      const __amdgpu_buffer_rsrc_t ru = buf_rsrc(a.u + (tok0 * a.H + h) * (long)V, (int)(((L - 1) * rsv + V) * 4));
      f32x16 aw[NJK], av[NJV];
#pragma unroll
      for (int j = 0; j < NJK; ++j) aw[j] = zero16();
#pragma unroll
      for (int j = 0; j < NJV; ++j) av[j] = zero16();
#pragma unroll
      for (int s0 = 0; s0 < BT; s0 += 16) {
        const bf16x8 bh = frag_rm(sBh + tr * 32 * PT + s0, PT), bl = frag_rm(sBl + tr * 32 * PT + s0, PT);
        const bf16x8 ch = frag_rm(sCh + tr * 32 * PT + s0, PT), cl = frag_rm(sCl + tr * 32 * PT + s0, PT);
#pragma unroll
        for (int j = 0; j < NJK; ++j) {
          const bf16x8 kt = frag32_tr(sK + s0 * PK + ((w & 1) * NJK + j) * 32, PK);
          aw[j] = mfma(kt, bh, aw[j]);
          aw[j] = mfma(kt, bl, aw[j]);
        }
#pragma unroll
        for (int j = 0; j < NJV; ++j) {
          const bf16x8 vt = frag32_tr(sV + s0 * PV + ((w & 1) * NJV + j) * 32, PV);
          av[j] = mfma(vt, ch, av[j]);
          av[j] = mfma(vt, cl, av[j]);
        }
      }
      // the wave's tiles go through a private staging area in the A / T buffers (dead after P5) and
      // leave as whole rows: w hi / lo as [32][WK] bf16, then u as [32][WV] fp32 (pitch 68)
      constexpr int WK = NJK * 32, WV = NJV * 32, PS = 68;
      bf16* swh = (bf16*)((char*)(w < 2 ? sA : sTf) + (w & 1) * (32 * PS * 4));
      bf16* swl = swh + 32 * PS;
      float* su = (float*)swh;
      const int rl = acc_col();  // the lane's row within the wave's 32 rows
#pragma unroll
      for (int j = 0; j < NJK; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int kc = 32 * j + 8 * g + q4;
          bf16x4 hi4, lo4;
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            bf16 p, q;
            split2(aw[j][4 * g + ii], p, q);
            hi4[ii] = p;
            lo4[ii] = q;
          }
          *(bf16x4*)(swh + rl * PS + kc) = hi4;
          *(bf16x4*)(swl + rl * PS + kc) = lo4;
        }
      {
        constexpr int LPR = WK / 8, RPI = 64 / LPR;  // lanes per row, rows per instruction
        const int c = 8 * (l % LPR), kbase = (w & 1) * WK;
#pragma unroll
        for (int rep = 0; rep < 32 / RPI; ++rep) {
          const int t = RPI * rep + l / LPR;
          const int off = (int)(((tr * 32 + t) * rsk + kbase + c) * 2);
          const bf16x8 hv = __builtin_shufflevector(*(const bf16x4*)(swh + t * PS + c),
                                                    *(const bf16x4*)(swh + t * PS + c + 4), 0, 1, 2, 3, 4, 5, 6, 7);
          const bf16x8 lv = __builtin_shufflevector(*(const bf16x4*)(swl + t * PS + c),
                                                    *(const bf16x4*)(swl + t * PS + c + 4), 0, 1, 2, 3, 4, 5, 6, 7);
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, hv), rw, off, 0, 0);
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, lv), rwl, off, 0, 0);
        }
      }
#pragma unroll
      for (int j = 0; j < NJV; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int vc = 32 * j + 8 * g + q4;
          *(f32x4*)(su + rl * PS + vc) = f32x4{av[j][4 * g], av[j][4 * g + 1], av[j][4 * g + 2], av[j][4 * g + 3]};
        }
      {
        constexpr int LPR = WV / 4, RPI = 64 / LPR;
        const int c = 4 * (l % LPR), vbase = (w & 1) * WV;
#pragma unroll
        for (int rep = 0; rep < 32 / RPI; ++rep) {
          const int t = RPI * rep + l / LPR;
          const f32x4 x = *(const f32x4*)(su + t * PS + c);
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), ru,
                                                 (int)(((tr * 32 + t) * rsv + vbase + c) * 4), 0, 0);
        }
      }
    }
    __syncthreads();  // B7: k, v, g, beta free for the next unit
  }
}

// ===========================================================================
// gdn_fwd_state: grid ((V/32) * N * H)
// ===========================================================================
template <int K>
__global__ __launch_bounds__(kThreads) void gdn_fwd_state_kernel(const GdnArgs a, const int V) {
  constexpr int VB = 32, LDK = K + 8, LDKR = K + 16, LDU = BT + 4, LDV = VB + 4, NRT = K / 32, TPW = (NRT + 3) / 4;
  __shared__ __attribute__((aligned(16))) bf16 sW[BT * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sWl[BT * LDK];
  // k rows [t][k] (row-major: whole 16-byte writes; the state update reads K^T by transposing reads)
  __shared__ __attribute__((aligned(16))) bf16 sK[BT * LDKR];
  __shared__ __attribute__((aligned(16))) bf16 sST[VB * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sSTl[VB * LDK];
  __shared__ __attribute__((aligned(16))) float sU[BT * LDV];
  __shared__ __attribute__((aligned(16))) float sUsT[VB * LDU];  // (fac U)^T, rows read as 16-byte pieces
  __shared__ float sFac[BT];
  __shared__ float sGL[1];

  const int tid = threadIdx.x, w = wave_id();
  const int nv = V / VB;
  int unit, vt;
  xcd_map(blockIdx.x, nv, a.N * a.H, unit, vt);
  const int n = unit / a.H, h = unit % a.H;
  long bos;
  int len;
  seq_bounds(a.cu, n, a.T, bos, len);
  const int nc = (len + BT - 1) / BT;
  const int gc0 = a.cu ? a.chunk_off[n] : n * a.NT;
  const int v0 = vt * VB;
  const long rsk = (long)a.H * K, rsv = (long)a.H * V;

  f32x16 S[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    S[j] = zero16();
    const int rt = w + 4 * j;
    if (rt < NRT && a.s0) {
#pragma unroll
      for (int i = 0; i < 16; ++i) S[j][i] = a.s0[((long)unit * K + rt * 32 + acc_row(i)) * V + v0 + acc_col()];
    }
  }

  // Everything a step reads except the state itself is loaded one step ahead into registers.
  PrefetchBf16<K, BT> pw, pwl, pk;
  PrefetchF32<VB, BT> pu;
  float pg = 0.f, pgl = 0.f;
  auto issue = [&](int c) {
    const int c0 = c * BT, L = min(BT, len - c0);
    const long tok0 = bos + c0;
    pw.load((const bf16*)a.w + (tok0 * a.H + h) * K, rsk, L);
    pwl.load((const bf16*)a.wl + (tok0 * a.H + h) * K, rsk, L);
    pk.load((const bf16*)a.k + (tok0 * a.H + h) * K, rsk, L);
    pu.load(a.u + (tok0 * a.H + h) * (long)V + v0, rsv, L);
    if (tid < BT) {
      pgl = a.gcum[(tok0 + L - 1) * a.H + h];
      pg = (tid < L) ? a.gcum[(tok0 + tid) * a.H + h] : pgl;
    }
  };
  if (nc > 0) issue(0);

  for (int c = 0; c < nc; ++c) {
    const int c0 = c * BT, L = min(BT, len - c0), gc = gc0 + c;
    const long tok0 = bos + c0;
    pw.store(sW, LDK, nullptr, 0);
    pwl.store(sWl, LDK, nullptr, 0);
    pk.store(sK, LDKR, nullptr, 0);
    pu.store(sU, LDV, nullptr, 0);
    if (tid < BT) {
      sFac[tid] = __expf(pgl - pg);
      if (tid == 0) sGL[0] = __expf(pgl);
    }
    // S^T (hi/lo) as 8-byte pieces of four consecutive state rows
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int rt = w + 4 * j;
      if (rt < NRT) acc_to_lds_t(S[j], sST, sSTl, LDK, rt * 32);
    }
    __syncthreads();
    // the next chunk's loads: waves 2-3 (which store the snapshot) at once, waves 0-1 after their
    // products (issuing them first held the products behind a stalled memory queue)
    if (w >= 2 && c + 1 < nc) issue(c + 1);
    if (w < 2) {
      f32x16 acc = zero16();
      // w S with both operands as hi/lo pairs (lo x lo dropped)
      mma_rr(acc, sW + w * 32 * LDK, LDK, sST, LDK, K);
      mma_rr(acc, sW + w * 32 * LDK, LDK, sSTl, LDK, K);
      mma_rr(acc, sWl + w * 32 * LDK, LDK, sST, LDK, K);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = w * 32 + acc_row(i), cc = acc_col();
        float us = 0.f;
        if (r < L) {
          const float uu = sU[r * LDV + cc] - acc[i];
          sU[r * LDV + cc] = uu;  // U rows leave from LDS after the barrier
          us = sFac[r] * uu;
        }
        sUsT[cc * LDU + r] = us;
      }
      if (c + 1 < nc) issue(c + 1);
    } else {
      // state snapshot to HBM for the output kernel and the backward: int16 rows with a scale per
      // row (a row's K / 8 lanes are an aligned lane group of waves 2-3), else hi/lo pairs
      constexpr int VPR = K / 8;
      if (a.snap16 & 1) {
#pragma unroll
        for (int j = 0; j < (VB * VPR) / 128; ++j) {
          const int idx = tid - 128 + j * 128, r = idx / VPR, cc = (idx % VPR) * 8;
          const long row = ((long)gc * a.H + h) * V + v0 + r;
          snap16_store<K>(sST + r * LDK + cc, sSTl + r * LDK + cc, (short*)a.hT + row * K + cc, (float*)a.hTl + row,
                          tid);
        }
      } else {
        for (int idx = tid - 128; idx < 2 * VB * VPR; idx += 128) {
          const int which = idx / (VB * VPR), e = idx % (VB * VPR);
          const int r = e / VPR, cc = (e % VPR) * 8;
          const bf16* src = which ? sSTl : sST;
          bf16* dst = which ? (bf16*)a.hTl : (bf16*)a.hT;
          *(bf16x8*)(dst + (((long)gc * a.H + h) * V + v0 + r) * K + cc) = *(const bf16x8*)(src + r * LDK + cc);
        }
      }
    }
    __syncthreads();
    // U rows of the chunk to HBM as 16-byte pieces
#pragma unroll
    for (int j = 0; j < (BT * VB / 4) / kThreads; ++j) {
      const int idx = tid + j * kThreads, r = idx / (VB / 4), c4 = (idx % (VB / 4)) * 4;
      if (r < L) *(f32x4*)(a.U + (tok0 + r) * rsv + (long)h * V + v0 + c4) = *(const f32x4*)(sU + r * LDV + c4);
    }
    const float gL = sGL[0];
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int rt = w + 4 * j;
      if (rt < NRT) {
#pragma unroll
        for (int i = 0; i < 16; ++i) S[j][i] *= gL;
        for (int k0 = 0; k0 < BT; k0 += 16) {
          const bf16x8 ka = frag32_tr(sK + k0 * LDKR + rt * 32, LDKR);
          bf16x8 hi, lo;
          frag_rm_f32(sUsT + k0, LDU, hi, lo);
          S[j] = mfma(ka, hi, S[j]);
          S[j] = mfma(ka, lo, S[j]);
        }
      }
    }
    __syncthreads();
  }
  if (a.s_fin) {
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int rt = w + 4 * j;
      if (rt < NRT) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
          a.s_fin[((long)unit * K + rt * 32 + acc_row(i)) * V + v0 + acc_col()] = S[j][i];
      }
    }
  }
}


// ===========================================================================
// gdn_fwd_state for K <= 128 with 8 wavefronts, with the chunk output fused in: waves 0-3 compute
// and issue no global access inside the walk; waves 4-7 move memory one or two chunks ahead of its
// use and write every result row.  Compute wave w owns query / U rows [16 w, 16 w + 16) of every
// chunk.  Per chunk c:
//   phase A  compute: U = u - w S and Y = Qc S with the previous state (16x16 tiles, hi/lo
//                     operands sharing the state fragments); U over u in LDS, (fac U)^T and U^T
//                     (hi/lo) to LDS; the Qc fragments stay in registers
//            memory:  k of c+1 to LDS (k and g in two buffers by chunk parity); loads of k(c+2);
//                     state snapshot S_c and the output rows of c-1 to HBM
//   phase B  compute: S <- gamma_L S + K^T diag(fac) U (K^T fragments by transposing LDS reads),
//                     S^T (hi/lo) to LDS for chunk c+1; P^T = K Qc^T for the wave's rows, masked to
//                     s <= t and scaled by scale exp(g_t - g_s) (to HBM, one key tile per value
//                     block); O = scale gamma_t Y + P U to LDS (bf16)
//            memory:  U rows of c to HBM; w, wl, Qc (hi/lo), u, g of c+1 to LDS; loads of Qc(c+2)
//                     and w, wl, u, g(c+3)
// P never leaves the registers of the wave that forms it: its C tiles (lane = query row, four key
// rows per lane group) feed the A operand of P U directly, with the contraction index permuted the
// same way in the U^T operand (two 8-byte reads per lane).  Result rows leave through LDS as whole
// 16-byte pieces: scattered 2- and 4-byte stores from the compute waves stall the shared
// vector-memory path.
// LDS pitches: tiles read as mfma16 operands are K + 16 (or 64 + 16) elements wide, which keeps those
// reads free of bank conflicts; rows are written by 16 consecutive lanes per row.  For K = 128 the
// buffers fill the 160 KiB of LDS.
// ===========================================================================
// S16: the state snapshots leave as int16 rows with row scales (else hi/lo pairs)
template <int K, bool Q32, bool S16>
__global__ __launch_bounds__(kWalk8) void gdn_fwd_state_v3_kernel(const GdnArgs a, const int V) {
  constexpr int VB = 32, LDK = K + 16, LDB = BT + 16, LDV = VB + 4, LDO = VB + 4;
  constexpr int NM = 256;               // memory threads
  constexpr int RW = K / 4, NR16 = RW / 16;  // S rows per compute wave, in 16-row tiles
  constexpr int NK32 = K / 32, NT16 = BT / 16;
  __shared__ __attribute__((aligned(16))) bf16 sW[BT * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sWl[BT * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sQh[BT * LDK];   // Qc [t][k], hi
  __shared__ __attribute__((aligned(16))) bf16 sQl[BT * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sK[2 * BT * LDK];  // k [t][k], by chunk parity
  __shared__ __attribute__((aligned(16))) bf16 sSh[VB * LDK];   // S^T [v][k], hi
  __shared__ __attribute__((aligned(16))) bf16 sSl[VB * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sUh[VB * LDB];   // (fac U)^T [v][t], hi
  __shared__ __attribute__((aligned(16))) bf16 sUl[VB * LDB];
  __shared__ __attribute__((aligned(16))) bf16 sVh[VB * LDB];   // U^T [v][t], hi
  __shared__ __attribute__((aligned(16))) bf16 sVl[VB * LDB];
  __shared__ __attribute__((aligned(16))) float sU[BT * LDV];   // u [t][v], then U
  __shared__ __attribute__((aligned(16))) bf16 sO[BT * LDO];    // O [t][v]
  __shared__ __attribute__((aligned(16))) float sG[2 * BT];     // g_t (the last token's beyond the chunk), by chunk parity

  // the wave index as a wave-uniform value: the role branches are then uniform, and the wait
  // counts of one role's memory operations never merge with the other role's path
  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(wave_id()), l = lane_id();
  const bool mem = w >= 4;
  const int lm = tid - NM;
  const int nv = V / VB;
  int unit, vt;
  xcd_map(blockIdx.x, nv, a.N * a.H, unit, vt);
  const int n = unit / a.H, h = unit % a.H;
  long bos;
  int len;
  seq_bounds(a.cu, n, a.T, bos, len);
  const int nc = (len + BT - 1) / BT;
  const int gc0 = a.cu ? a.chunk_off[n] : n * a.NT;
  const int v0 = vt * VB;
  const long rsk = (long)a.H * K, rsv = (long)a.H * V;
  auto chunk_len = [&](int c) { return min(BT, len - c * BT); };
  auto tok_of = [&](int c) { return bos + (long)c * BT; };

  // compute waves: state rows [RW w, RW w + RW) x 32 value columns as 16x16 tiles
  f32x4 S[NR16][2];
#pragma unroll
  for (int rt = 0; rt < NR16; ++rt)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) S[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};

  // memory waves: w, wl, u, g two chunks ahead in two register sets used by chunk parity; k and Qc
  // one chunk ahead
  RowsBf16<K, BT, NM> pw[2], pwl[2], pk;
  RowsF32<VB, BT, NM> pu[2];
  RowsF32<K, BT, NM> pq;
  float pg[2] = {0.f, 0.f};
  auto load_wug = [&](int c, auto P) {
    constexpr int p = decltype(P)::value;
    const int L = chunk_len(c);
    const long tok0 = tok_of(c);
    pw[p].load((const bf16*)a.w + (tok0 * a.H + h) * K, rsk, L, lm);
    pwl[p].load((const bf16*)a.wl + (tok0 * a.H + h) * K, rsk, L, lm);
    pu[p].load(a.u + (tok0 * a.H + h) * (long)V + v0, rsv, L, lm);
    pg[p] = a.gcum[(tok0 + min(lm & (BT - 1), L - 1)) * a.H + h];
  };
  auto load_q = [&](int c) {
    const long o = (tok_of(c) * a.H + h) * K;
    if (Q32)
      pq.load(a.qc32 + o, rsk, chunk_len(c), lm);
    else
      pq.load(nullptr, (const bf16*)a.qc16 + o, rsk, chunk_len(c), lm);
  };
  auto load_k = [&](int c) { pk.load((const bf16*)a.k + (tok_of(c) * a.H + h) * K, rsk, chunk_len(c), lm); };
  // w, wl, Qc, u, g of chunk c to LDS (lane t of every memory wave holds g of token t of the chunk;
  // wave 4 writes g); g goes to the buffer of the chunk's parity P
  auto stage_wug = [&](int c, auto P) {
    constexpr int p = decltype(P)::value;
    const int L = chunk_len(c);
    pw[p].store(sW, LDK, L, lm);
    pwl[p].store(sWl, LDK, L, lm);
    pq.store_split(sQh, sQl, LDK, L, lm);
    pu[p].store(sU, LDV, L, lm);
    if (w == 4) sG[p * BT + l] = pg[p];
  };
  // output rows of chunk c (bf16, 64 bytes per row and value block) from LDS to HBM: one 16-byte
  // piece per memory thread; rows past the chunk write row L - 1 again (same value, same address), so
  // every pass issues the same stores
  auto store_o = [&](int c) {
    const int r = min(lm >> 2, chunk_len(c) - 1), cc = (lm & 3) * 8;
    const bf16* src = sO + r * LDO + cc;
    typedef __bf16 b4 __attribute__((ext_vector_type(4)));
    const bf16x8 o8 = __builtin_shufflevector(*(const b4*)src, *(const b4*)(src + 4), 0, 1, 2, 3, 4, 5, 6, 7);
    *(bf16x8*)(gmem((bf16*)a.o) + (tok_of(c) + r) * rsv + (long)h * V + v0 + cc) = o8;
  };
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;

  // Each role runs its own loop (both pass the same 1 + 2 nc barriers), so the compiler's wait
  // counts for the memory waves follow their own sequence of operations only.  Loads and stores
  // are unconditional (the last chunk again past the end, row L - 1 again past the chunk): every
  // pass issues the same memory operations, so each wait counts exactly the younger ones.
  if (mem) {
    const int cl = nc - 1;
    if (nc > 0) {
      load_wug(0, P0{});
      load_q(0);
      load_k(0);
      load_wug(min(1, cl), P1{});
      stage_wug(0, P0{});
      pk.store(sK, LDK, chunk_len(0), lm);
      load_q(min(1, cl));
      load_k(min(1, cl));
      load_wug(min(2, cl), P0{});
    }
    __syncthreads();
    // chunk c with register set Q = (c + 1) % 2 (w, wl, u, g of chunk c + 1 on entry)
    auto chunk = [&](int c, auto Q) {
      constexpr int q = decltype(Q)::value;
      const int gc = gc0 + c, L = chunk_len(c);
      const long tok0 = tok_of(c);
      // ---- phase A: k of c+1 to its buffer; loads of k(c+2); snapshot S_c; output rows of c-1
      pk.store(sK + q * (BT * LDK), LDK, chunk_len(min(c + 1, cl)), lm);
      load_k(min(c + 2, cl));
      constexpr int VPR = K / 8;
      if constexpr (S16) {
#pragma unroll
        for (int j = 0; j < (VB * VPR) / NM; ++j) {
          const int idx = lm + j * NM, r = idx / VPR, cc = (idx % VPR) * 8;
          const long row = ((long)gc * a.H + h) * V + v0 + r;
          snap16_store<K>(sSh + r * LDK + cc, sSl + r * LDK + cc, (short*)a.hT + row * K + cc, (float*)a.hTl + row, lm);
        }
      } else {
#pragma unroll
        for (int j = 0; j < (2 * VB * VPR) / NM; ++j) {
          const int idx = lm + j * NM;
          const int which = idx / (VB * VPR), e = idx % (VB * VPR);
          const int r = e / VPR, cc = (e % VPR) * 8;
          const bf16* src = which ? sSl : sSh;
          bf16* dst = which ? (bf16*)a.hTl : (bf16*)a.hT;
          *(bf16x8*)(gmem(dst) + (((long)gc * a.H + h) * V + v0 + r) * K + cc) = *(const bf16x8*)(src + r * LDK + cc);
        }
      }
      store_o(max(c - 1, 0));
      __syncthreads();
      // ---- phase B: U rows of c (read before u of c+1 replaces them: each thread reads exactly the
      // pieces it overwrites), w, wl, Qc, u, g of c+1; loads of Qc(c+2) and w, wl, u, g(c+3)
      constexpr int NU = (BT * VB / 4) / NM;
      f32x4 urow[NU];
#pragma unroll
      for (int j = 0; j < NU; ++j) {
        const int idx = lm + j * NM, r = idx / (VB / 4), cc = (idx % (VB / 4)) * 4;
        urow[j] = *(const f32x4*)(sU + min(r, L - 1) * LDV + cc);
      }
      stage_wug(min(c + 1, cl), Q);
#pragma unroll
      for (int j = 0; j < NU; ++j) {
        const int idx = lm + j * NM, r = min(idx / (VB / 4), L - 1), cc = (idx % (VB / 4)) * 4;
        *(f32x4*)(gmem(a.U) + (tok0 + r) * rsv + (long)h * V + v0 + cc) = urow[j];
      }
      load_q(min(c + 2, cl));
      load_wug(min(c + 3, cl), Q);
      __syncthreads();
    };
    // pairs of chunks, then the odd one: the loop is entered again only after an odd chunk, so
    // the register sets hold the same chunks at every pass
    int c = 0;
    for (; c + 1 < nc; c += 2) {
      chunk(c, P1{});
      chunk(c + 1, P0{});
    }
    if (c < nc) chunk(c, P1{});
    // the last chunk's output rows (written before the last barrier)
    if (nc > 0) store_o(nc - 1);
    return;
  }

  // compute waves
  if (a.s0) {
#pragma unroll
    for (int rt = 0; rt < NR16; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          S[rt][ct][i] = a.s0[((long)unit * K + RW * w + 16 * rt + 4 * (l >> 4) + i) * V + v0 + 16 * ct + (l & 15)];
  }
#pragma unroll
  for (int rt = 0; rt < NR16; ++rt)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) acc16_to_lds_t(S[rt][ct], sSh + 16 * ct * LDK, sSl + 16 * ct * LDK, LDK, RW * w + 16 * rt);
  __syncthreads();
  const int rb = 16 * w + 4 * (l >> 4);  // first of the lane's four rows in C tiles of this wave's rows
  const int tq = 16 * w + (l & 15);      // the lane's query row in P^T tiles
  for (int c = 0; c < nc; ++c) {
    const int L = chunk_len(c), gc = gc0 + c;
    const bf16* sKc = sK + (c & 1) * (BT * LDK);
    const float* sGc = sG + (c & 1) * BT;
    // ---- phase A: U = u - w S and Y = Qc S, both with hi/lo operands (lo x lo dropped)
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    f32x4 y[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    bf16x8 qh[NK32], ql[NK32];
#pragma unroll
    for (int kk = 0; kk < NK32; ++kk) {
      const int k0 = 32 * kk;
      const bf16x8 wh = frag16_rm(sW + 16 * w * LDK + k0, LDK), wl = frag16_rm(sWl + 16 * w * LDK + k0, LDK);
      qh[kk] = frag16_rm(sQh + 16 * w * LDK + k0, LDK);
      ql[kk] = frag16_rm(sQl + 16 * w * LDK + k0, LDK);
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        const bf16x8 sh = frag16_rm(sSh + 16 * ct * LDK + k0, LDK);
        const bf16x8 sl = frag16_rm(sSl + 16 * ct * LDK + k0, LDK);
        acc[ct] = mfma16(wh, sh, acc[ct]);
        acc[ct] = mfma16(wh, sl, acc[ct]);
        acc[ct] = mfma16(wl, sh, acc[ct]);
        y[ct] = mfma16(qh[kk], sh, y[ct]);
        y[ct] = mfma16(qh[kk], sl, y[ct]);
        y[ct] = mfma16(ql[kk], sh, y[ct]);
      }
    }
    // g of the lane's rows and of the chunk's last token; fac_t = exp(g_L - g_t), 0 beyond the chunk
    // (rows beyond the chunk hold u = 0 and w = 0, so U = 0 there and fac = 0 keeps it out of S)
    const float glast = sGc[L - 1];
    const float gL = __expf(glast);
    const f32x4 gr = *(const f32x4*)(sGc + rb);
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const int cc = 16 * ct + (l & 15);
      f32x4 uo, us;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float* pu_ = sU + (rb + i) * LDV + cc;
        uo[i] = *pu_ - acc[ct][i];
        *pu_ = uo[i];
        us[i] = rb + i < L ? __expf(glast - gr[i]) * uo[i] : 0.f;
      }
      acc16_to_lds_t(us, sUh + 16 * ct * LDB, sUl + 16 * ct * LDB, LDB, 16 * w);
      acc16_to_lds_t(uo, sVh + 16 * ct * LDB, sVl + 16 * ct * LDB, LDB, 16 * w);
    }
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int i = 0; i < 4; ++i) y[ct][i] *= a.scale * __expf(gr[i]);
    __syncthreads();

    // ---- phase B: S <- gamma_L S + K^T (fac U); S^T (hi/lo) for the next chunk
#pragma unroll
    for (int rt = 0; rt < NR16; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) S[rt][ct] *= gL;
#pragma unroll
    for (int k0 = 0; k0 < BT; k0 += 32) {
      bf16x8 uh[2], ul[2];
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        uh[ct] = frag16_rm(sUh + 16 * ct * LDB + k0, LDB);
        ul[ct] = frag16_rm(sUl + 16 * ct * LDB + k0, LDB);
      }
#pragma unroll
      for (int rt = 0; rt < NR16; ++rt) {
        const bf16x8 ka = frag16_tr(sKc + k0 * LDK + RW * w + 16 * rt, LDK);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
          S[rt][ct] = mfma16(ka, uh[ct], S[rt][ct]);
          S[rt][ct] = mfma16(ka, ul[ct], S[rt][ct]);
        }
      }
    }
    // P^T tiles of key rows [16 i, 16 i + 16) against this wave's query rows (causal: i <= w), with
    // the query fragments kept from phase A
    f32x4 pt[NT16];
#pragma unroll
    for (int i = 0; i < NT16; ++i) {
      pt[i] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (i <= w) {
#pragma unroll
        for (int kk = 0; kk < NK32; ++kk) {
          const bf16x8 kf = frag16_rm(sKc + 16 * i * LDK + 32 * kk, LDK);
          pt[i] = mfma16(kf, qh[kk], pt[i]);
          pt[i] = mfma16(kf, ql[kk], pt[i]);
        }
      }
    }
    // P[t][s] = scale exp(g_t - g_s) (Qc_t . k_s) for s <= t < L, else 0 (the exponent is taken
    // only where it is used, so masked entries never overflow)
    const float gq = sGc[tq];
#pragma unroll
    for (int i = 0; i < NT16; ++i) {
      const f32x4 gs = *(const f32x4*)(sGc + 16 * i + 4 * (l >> 4));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool keep = 16 * i + 4 * (l >> 4) + j <= tq && tq < L;
        const float e = __expf(keep ? gq - gs[j] : 0.f);
        pt[i][j] = keep ? a.scale * e * pt[i][j] : 0.f;
      }
    }
    // P^T to HBM: every value block forms the whole tile; block vt writes the key tiles i with
    // i % nv == vt (64-byte rows)
    {
      float* ptg = a.PT + ((long)gc * a.H + h) * (BT * BT);
#pragma unroll
      for (int i = 0; i < NT16; ++i)
        if (i % nv == vt) {
#pragma unroll
          for (int j = 0; j < 4; ++j) ptg[(16 * i + 4 * (l >> 4) + j) * BT + tq] = pt[i][j];
        }
    }
    // A operands of P U: k slots 0-3 from key tile 2p, 4-7 from key tile 2p + 1
    bf16x8 ph[NT16 / 2], pl[NT16 / 2];
#pragma unroll
    for (int p = 0; p < NT16 / 2; ++p)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bf16 x, z;
        split2(pt[2 * p][j], x, z);
        ph[p][j] = x;
        pl[p][j] = z;
        split2(pt[2 * p + 1][j], x, z);
        ph[p][4 + j] = x;
        pl[p][4 + j] = z;
      }
    // O = scale gamma Y + P U over the key tiles this wave's rows see
#pragma unroll
    for (int p = 0; p < NT16 / 2; ++p) {
      if (2 * p <= w) {
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
          const int e = (16 * ct + (l & 15)) * LDB + 32 * p + 4 * (l >> 4);
          const bf16x8 vh = __builtin_shufflevector(*(const bf16x4*)(sVh + e), *(const bf16x4*)(sVh + e + 16), 0,
                                                    1, 2, 3, 4, 5, 6, 7);
          const bf16x8 vl = __builtin_shufflevector(*(const bf16x4*)(sVl + e), *(const bf16x4*)(sVl + e + 16), 0,
                                                    1, 2, 3, 4, 5, 6, 7);
          y[ct] = mfma16(ph[p], vh, y[ct]);
          y[ct] = mfma16(ph[p], vl, y[ct]);
          y[ct] = mfma16(pl[p], vh, y[ct]);
        }
      }
    }
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int i = 0; i < 4; ++i) sO[(rb + i) * LDO + 16 * ct + (l & 15)] = (bf16)y[ct][i];
#pragma unroll
    for (int rt = 0; rt < NR16; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
        acc16_to_lds_t(S[rt][ct], sSh + 16 * ct * LDK, sSl + 16 * ct * LDK, LDK, RW * w + 16 * rt);
    __syncthreads();
  }
  if (a.s_fin) {
#pragma unroll
    for (int rt = 0; rt < NR16; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          a.s_fin[((long)unit * K + RW * w + 16 * rt + 4 * (l >> 4) + i) * V + v0 + 16 * ct + (l & 15)] = S[rt][ct][i];
  }
}

// ===========================================================================
// gdn_fwd_o: grid (NTG, H)
// ===========================================================================
// S16: the state snapshots are int16 rows with a scale per row (else hi/lo pairs)
template <int K, bool S16>
__global__ __launch_bounds__(kThreads) void gdn_fwd_o_kernel(const GdnArgs a, const int V) {
  constexpr int LDQ = K + 4, LDK = K + 8, LDP = BT + 1;
  // the state is staged as a hi/lo pair per 64 value columns x KS key rows
  constexpr int KS = K > 128 ? 128 : K, NKS = K / KS, LDS_ = KS + 8;
  constexpr long kRegion = (long)BT * LDK * 2 > 2L * 64 * LDS_ * 2 ? (long)BT * LDK * 2 : 2L * 64 * LDS_ * 2;
  constexpr long kBytes = (long)BT * LDQ * 4 + kRegion + 2L * BT * LDP * 4 + 2 * BT * 4 + 64;
  __shared__ __attribute__((aligned(16))) char smem[kBytes];
  Carver cv{smem};
  float* sQc = cv.take<float>(BT * LDQ);
  char* region = cv.p;
  cv.p += kRegion;
  bf16* sK = (bf16*)region;                 // K rows first; then the state tiles
  bf16* sHt = (bf16*)region;                // [64 v][KS] hi
  bf16* sHtl = sHt + 64 * LDS_;             // [64 v][KS] lo
  float* sP = cv.take<float>(BT * LDP);
  float* sUT = cv.take<float>(BT * LDP);
  float* sG = cv.take<float>(BT);
  float* sGam = cv.take<float>(BT);

  const int tid = threadIdx.x, w = wave_id();
  const int gc = blockIdx.x, h = blockIdx.y;
  int n, c0, L;
  long bos;
  if (!chunk_info(a, gc, n, c0, bos, L)) return;
  const long tok0 = bos + c0;
  const long rsk = (long)a.H * K, rsv = (long)a.H * V;

  // state slice (hi/lo) of step `it` = (value block it / NKS, key slice it % NKS) and, at a new value
  // block, its U, one step ahead
  PrefetchBf16<KS, 64> pS;
  PrefetchBf16<S16 ? 8 : KS, S16 ? 1 : 64> pSl;  // the lo parts (hi/lo snapshots only)
  float sc[PrefetchBf16<KS, 64>::N];              // row scales (int16 snapshots)
  PrefetchF32<64, BT> pU;
  auto issue = [&](int it) {
    const int v0 = (it / NKS) * 64, ks = (it % NKS) * KS;
    const long so = (((long)gc * a.H + h) * V + v0) * K + ks;
    pS.load((const bf16*)a.hT + so, K, 64);
    if constexpr (S16)
      pS.load_scales((const float*)a.hTl + ((long)gc * a.H + h) * V + v0, 64, sc);
    else
      pSl.load((const bf16*)a.hTl + so, K, 64);
    if (ks == 0) pU.load(a.U + (tok0 * a.H + h) * (long)V + v0, rsv, L);
  };
  issue(0);
  stage_any_f32<K>(sQc, LDQ, nullptr, 0, a.qc32 ? a.qc32 + (tok0 * a.H + h) * K : nullptr,
                   a.qc16 ? (const bf16*)a.qc16 + (tok0 * a.H + h) * K : nullptr, rsk, BT, L);
  stage_bf16<K>(sK, LDK, nullptr, 0, (const bf16*)a.k + (tok0 * a.H + h) * K, rsk, BT, L);
  if (tid < BT) {
    const float gl = a.gcum[(tok0 + L - 1) * a.H + h];
    const float gt = (tid < L) ? a.gcum[(tok0 + tid) * a.H + h] : gl;
    sG[tid] = gt;
    sGam[tid] = __expf(gt);
  }
  __syncthreads();

  float* ptg = a.PT + ((long)gc * a.H + h) * (BT * BT);
  if (w < 3) {
    const int tr = (w == 0) ? 0 : 1, tc = (w == 2) ? 1 : 0;
    f32x16 acc = zero16();
    for (int k0 = 0; k0 < K; k0 += 16) {
      bf16x8 hi, lo;
      frag_rm_f32(sQc + tr * 32 * LDQ + k0, LDQ, hi, lo);
      const bf16x8 b = frag_rm(sK + tc * 32 * LDK + k0, LDK);
      acc = mfma(hi, b, acc);
      acc = mfma(lo, b, acc);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = tr * 32 + acc_row(i), c = tc * 32 + acc_col();
      const float p = (r >= c && r < L) ? a.scale * __expf(sG[r] - sG[c]) * acc[i] : 0.f;
      sP[r * LDP + c] = p;
      ptg[c * BT + r] = p;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = acc_row(i), c = 32 + acc_col();
      sP[r * LDP + c] = 0.f;
      ptg[c * BT + r] = 0.f;
    }
  }
  __syncthreads();

  bf16* og = (bf16*)a.o + (tok0 * a.H + h) * (long)V;
  const int nit = (V / 64) * NKS;
  const int tr = w >> 1, tc = w & 1;
  f32x16 acc = zero16();
  for (int it = 0; it < nit; ++it) {
    const int v0 = (it / NKS) * 64, ks = (it % NKS) * KS;
    if constexpr (S16) {
      pS.store_s16_split(sHt, sHtl, LDS_, sc);
    } else {
      pS.store(sHt, LDS_, nullptr, 0);
      pSl.store(sHtl, LDS_, nullptr, 0);
    }
    if (ks == 0) pU.store(nullptr, 0, sUT, LDP);
    __syncthreads();
    if (it + 1 < nit) issue(it + 1);
    if (ks == 0) acc = zero16();
    for (int k0 = 0; k0 < KS; k0 += 16) {
      bf16x8 hi, lo;
      frag_rm_f32(sQc + tr * 32 * LDQ + ks + k0, LDQ, hi, lo);
      const bf16x8 bh = frag_rm(sHt + tc * 32 * LDS_ + k0, LDS_);
      const bf16x8 bl = frag_rm(sHtl + tc * 32 * LDS_ + k0, LDS_);
      acc = mfma(hi, bh, acc);
      acc = mfma(hi, bl, acc);
      acc = mfma(lo, bh, acc);
    }
    if (ks + KS < K) {
      __syncthreads();
      continue;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] *= a.scale * sGam[tr * 32 + acc_row(i)];
    for (int k0 = 0; k0 < BT; k0 += 16) {
      bf16x8 phi, plo, uhi, ulo;
      frag_rm_f32(sP + tr * 32 * LDP + k0, LDP, phi, plo);
      frag_rm_f32(sUT + tc * 32 * LDP + k0, LDP, uhi, ulo);
      acc = mfma(phi, uhi, acc);
      acc = mfma(phi, ulo, acc);
      acc = mfma(plo, uhi, acc);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = tr * 32 + acc_row(i);
      if (r < L) og[(long)r * rsv + v0 + tc * 32 + acc_col()] = (bf16)acc[i];
    }
    __syncthreads();
  }
}

// ===========================================================================
// gdn_bwd_state: grid ((V/32) * N * H), reverse walk
//   dU = P^T dO + diag(gamma_L/gamma) K dS'
//   dS <- gamma_L dS' + Qc^T diag(scale gamma) dO - w^T dU
// ===========================================================================
// Q32: q_clean arrives in fp32 (else bf16), a template parameter so that only one set of prefetch
// registers exists.
template <int K, bool Q32>
__global__ __launch_bounds__(kThreads) void gdn_bwd_state_kernel(const GdnArgs a, const int V) {
  constexpr int VB = 32, LDK = K + 8, LDP = BT + 1, NRT = K / 32, TPW = (NRT + 3) / 4;
  // query / w columns staged per pass of the dS update: 128 (four 32-row tiles, one per wave)
  constexpr int KH = K > 128 ? 128 : K, NKH = K / KH;
  // row-major tiles read as transposed operands (transposing LDS reads): pitches of 16-element
  // multiples plus 16
  constexpr int LDO = VB + 16, LDW = KH + 16, LDG = BT + 8;
  auto r16 = [](long b) { return (b + 15) & ~15L; };
  // k (the dU phase) and the query / w slices (the dS passes, K > 128) are never live together: one
  // region (with a single pass the slices are staged beside k at the chunk start)
  constexpr bool kAlias = NKH > 1;
  constexpr long kK = (((long)BT * LDK * 2) + 15) & ~15L;
  constexpr long kQW = 4 * ((((long)BT * LDW * 2) + 15) & ~15L);
  constexpr long kRegion = kAlias ? (kK > kQW ? kK : kQW) : kK + kQW;
  constexpr long kBytes = (long)BT * LDP * 4 + (long)BT * LDO * 2 + kRegion + (long)VB * LDK * 2 +
                          (long)VB * LDP * 4 + 4L * VB * LDG * 2 + 3L * BT * 4 + (long)VB * LDK * 2 + 16 * 16;
  __shared__ __attribute__((aligned(16))) char smem[kBytes];
  Carver cv{smem};
  float* sPT = cv.take<float>(BT * LDP);
  bf16* sdO = cv.take<bf16>(BT * LDO);      // dO [t][v]
  char* region = cv.p;
  cv.p += kRegion;
  bf16* sK = (bf16*)region;                 // k [t][k] (dU phase)
  // (dS passes) Qc and w slices [t][k slice] as hi/lo pairs, read as transposed operands
  bf16* sQh = (bf16*)(region + (kAlias ? 0 : kK));
  bf16* sQl = sQh + r16((long)BT * LDW * 2) / 2;
  bf16* sW = sQl + r16((long)BT * LDW * 2) / 2;
  bf16* sWl = sW + r16((long)BT * LDW * 2) / 2;
  bf16* sdST = cv.take<bf16>(VB * LDK);
  bf16* sdSTl = cv.take<bf16>(VB * LDK);
  float* sdUT = cv.take<float>(VB * LDP);   // -dU, [v][t] (for the dU rows to HBM)
  bf16* sdUh = cv.take<bf16>(VB * LDG);     // -dU, [v][t], hi / lo (operands)
  bf16* sdUl = cv.take<bf16>(VB * LDG);
  bf16* sgOh = cv.take<bf16>(VB * LDG);     // scale gamma_t dO[t][v], [v][t], hi / lo
  bf16* sgOl = cv.take<bf16>(VB * LDG);
  float* sFac = cv.take<float>(BT);
  float* sGam = cv.take<float>(BT);
  float* sGL = cv.take<float>(4);

  const int tid = threadIdx.x, w = wave_id();
  const int nv = V / VB;
  int unit, vt;
  xcd_map(blockIdx.x, nv, a.N * a.H, unit, vt);
  const int n = unit / a.H, h = unit % a.H;
  long bos;
  int len;
  seq_bounds(a.cu, n, a.T, bos, len);
  const int nc = (len + BT - 1) / BT;
  const int gc0 = a.cu ? a.chunk_off[n] : n * a.NT;
  const int v0 = vt * VB;
  const long rsk = (long)a.H * K, rsv = (long)a.H * V;

  f32x16 dS[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    dS[j] = zero16();
    const int rt = w + 4 * j;
    if (rt < NRT && a.ds_fin) {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        dS[j][i] = a.ds_fin[((long)unit * K + rt * 32 + acc_row(i)) * V + v0 + acc_col()];
    }
  }

  // Everything a step reads except dS itself is loaded one step ahead into registers.  For K = 256
  // the query / w rows go through LDS in KH-column slices (one slice per pass of the dS update);
  // each slice is loaded one pass ahead (the next chunk's first slice during the last pass).
  constexpr bool kPreQW = (NKH == 1);
  PrefetchF32<BT, BT> pP;
  PrefetchBf16<VB, BT> pO;
  PrefetchBf16<K, BT> pK;
  using QPre = typename std::conditional<Q32, PrefetchF32<KH, BT>, PrefetchBf16<KH, BT>>::type;
  QPre pQ;
  PrefetchBf16<KH, BT> pW, pWl;
  auto issue_qw = [&](int cc, int hb) {
    const int cx = cc * BT, Lx = min(BT, len - cx);
    const long tx = ((bos + cx) * a.H + h) * K + hb * KH;
    if constexpr (Q32) pQ.load(a.qc32 + tx, rsk, Lx);
    else pQ.load((const bf16*)a.qc16 + tx, rsk, Lx);
    pW.load((const bf16*)a.w + tx, rsk, Lx);
    pWl.load((const bf16*)a.wl + tx, rsk, Lx);
  };
  // Qc slice [t][k] as hi/lo bf16 (rows past the chunk were loaded as zeros)
  auto store_q = [&]() {
    if constexpr (Q32) {
      constexpr int VPR = KH / 4;
#pragma unroll
      for (int j = 0; j < QPre::N; ++j) {
        const int idx = threadIdx.x + j * kThreads;
        if (idx >= BT * VPR) continue;
        const int r = idx / VPR, c = (idx % VPR) * 4;
        bf16x4 hh, ll;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          bf16 x, y;
          split2(pQ.v[j][i], x, y);
          hh[i] = x;
          ll[i] = y;
        }
        *(bf16x4*)(sQh + r * LDW + c) = hh;
        *(bf16x4*)(sQl + r * LDW + c) = ll;
      }
    } else {
      constexpr int VPR = KH / 8;
#pragma unroll
      for (int j = 0; j < QPre::N; ++j) {
        const int idx = threadIdx.x + j * kThreads;
        if (idx >= BT * VPR) continue;
        const int r = idx / VPR, c = (idx % VPR) * 8;
        *(bf16x8*)(sQh + r * LDW + c) = pQ.v[j];
        *(bf16x8*)(sQl + r * LDW + c) = bf16x8{};
      }
    }
  };
  float pgl = 0.f, pgt = 0.f;
  auto issue = [&](int c) {
    const int c0 = c * BT, L = min(BT, len - c0), gc = gc0 + c;
    const long tok0 = bos + c0;
    pP.load(a.PT + ((long)gc * a.H + h) * (BT * BT), BT, BT);
    pO.load((const bf16*)a.dout + (tok0 * a.H + h) * (long)V + v0, rsv, L);
    pK.load((const bf16*)a.k + (tok0 * a.H + h) * K, rsk, L);
    if (kPreQW) issue_qw(c, 0);
    if (tid < BT) {
      pgl = a.gcum[(tok0 + L - 1) * a.H + h];
      pgt = (tid < L) ? a.gcum[(tok0 + tid) * a.H + h] : pgl;
    }
  };
  if (nc > 0) issue(nc - 1);
  if (!kPreQW && nc > 0) issue_qw(nc - 1, 0);

  for (int c = nc - 1; c >= 0; --c) {
    const int c0 = c * BT, L = min(BT, len - c0), gc = gc0 + c;
    const long tok0 = bos + c0;
    pP.store(sPT, LDP, nullptr, 0);
    pO.store(sdO, LDO, nullptr, 0);
    pK.store(sK, LDK, nullptr, 0);
    if (kPreQW) {
      store_q();
      pW.store(sW, LDW, nullptr, 0);
      pWl.store(sWl, LDW, nullptr, 0);
    }
    if (tid < BT) {
      sFac[tid] = __expf(pgl - pgt);
      sGam[tid] = (tid < L) ? __expf(pgt) : 0.f;
      if (tid == 0) sGL[0] = __expf(pgl);
    }
    // dS'^T (hi/lo) as 8-byte pieces of four consecutive state rows
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int rt = w + 4 * j;
      if (rt < NRT) acc_to_lds_t(dS[j], sdST, sdSTl, LDK, rt * 32);
    }
    __syncthreads();
    // the previous chunk's loads: waves 2-3 at once, waves 0-1 after their dU products (issued
    // first, a stalled memory queue held the products)
    if (w >= 2 && c > 0) issue(c - 1);
    if (a.snap16 & 2) {
      // int16 rows with a scale per row (a row's K / 8 lanes are an aligned lane group)
      constexpr int VPR = K / 8;
#pragma unroll
      for (int j = 0; j < (VB * VPR) / kThreads; ++j) {
        const int idx = tid + j * kThreads, r = idx / VPR, cc = (idx % VPR) * 8;
        const long row = ((long)gc * a.H + h) * V + v0 + r;
        snap16_store<K>(sdST + r * LDK + cc, sdSTl + r * LDK + cc, (short*)a.dhT + row * K + cc,
                        (float*)a.dhTl + row, tid);
      }
    } else {
      lds_to_global_bf16<K>((bf16*)a.dhT + (((long)gc * a.H + h) * V + v0) * K, K, sdST, LDK, VB);
      lds_to_global_bf16<K>((bf16*)a.dhTl + (((long)gc * a.H + h) * V + v0) * K, K, sdSTl, LDK, VB);
    }
    if (w < 2) {
      f32x16 acc = zero16(), acc2 = zero16();
      for (int k0 = 0; k0 < BT; k0 += 16) {
        bf16x8 hi, lo;
        frag_rm_f32(sPT + w * 32 * LDP + k0, LDP, hi, lo);
        const bf16x8 b = frag32_tr(sdO + k0 * LDO, LDO);
        acc = mfma(hi, b, acc);
        acc = mfma(lo, b, acc);
      }
      // K dS' with dS' as hi/lo: two independent accumulator chains
      f32x16 acc3 = zero16();
#pragma unroll 4
      for (int k0 = 0; k0 < K; k0 += 16) {
        const bf16x8 ka = frag_rm(sK + w * 32 * LDK + k0, LDK);
        acc2 = mfma(ka, frag_rm(sdST + k0, LDK), acc2);
        acc3 = mfma(ka, frag_rm(sdSTl + k0, LDK), acc3);
      }
      f32x16 ndu;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = w * 32 + acc_row(i), cc = acc_col();
        ndu[i] = r < L ? -(acc[i] + sFac[r] * (acc2[i] + acc3[i])) : 0.f;
        sdUT[cc * LDP + r] = ndu[i];  // dU rows leave from LDS after the barrier
      }
      acc_to_lds_t(ndu, sdUh, sdUl, LDG, w * 32);
      if (c > 0) issue(c - 1);
    } else {
      for (int e = tid - 128; e < VB * BT; e += 128) {
        const int vv = e / BT, t = e % BT;
        split2(a.scale * sGam[t] * (float)sdO[t * LDO + vv], sgOh[vv * LDG + t], sgOl[vv * LDG + t]);
      }
    }
    __syncthreads();
    // dU rows of the chunk to HBM as 16-byte pieces (from the negated transposed copy)
#pragma unroll
    for (int j = 0; j < (BT * VB / 4) / kThreads; ++j) {
      const int idx = tid + j * kThreads, r = idx / (VB / 4), c4 = (idx % (VB / 4)) * 4;
      if (r < L) {
        const f32x4 du = f32x4{-sdUT[c4 * LDP + r], -sdUT[(c4 + 1) * LDP + r], -sdUT[(c4 + 2) * LDP + r],
                               -sdUT[(c4 + 3) * LDP + r]};
        *(f32x4*)(a.dU + (tok0 + r) * rsv + (long)h * V + v0 + c4) = du;
      }
    }
    const float gL = sGL[0];
    for (int hb = 0; hb < NKH; ++hb) {
      if (!kPreQW) {
        // slice hb (loaded one pass ahead) into LDS; the next slice's loads
        store_q();
        pW.store(sW, LDW, nullptr, 0);
        pWl.store(sWl, LDW, nullptr, 0);
        if (hb + 1 < NKH) issue_qw(c, hb + 1);
        else if (c > 0) issue_qw(c - 1, 0);
        __syncthreads();
      }
#pragma unroll
      for (int j = 0; j < TPW; ++j) {
        const int rt = w + 4 * j;
        if (rt < NRT && (rt * 32) / KH == hb) {
          const int lr = rt * 32 - hb * KH;
#pragma unroll
          for (int i = 0; i < 16; ++i) dS[j][i] *= gL;
          // Qc^T (scale gamma dO) into dS, -w^T dU into a second accumulator chain
          f32x16 d2 = zero16();
#pragma unroll
          for (int k0 = 0; k0 < BT; k0 += 16) {
            const bf16x8 qh = frag32_tr(sQh + k0 * LDW + lr, LDW), ql = frag32_tr(sQl + k0 * LDW + lr, LDW);
            const bf16x8 gh = frag_rm(sgOh + k0, LDG), gl = frag_rm(sgOl + k0, LDG);
            const bf16x8 wa = frag32_tr(sW + k0 * LDW + lr, LDW), wal = frag32_tr(sWl + k0 * LDW + lr, LDW);
            const bf16x8 dh = frag_rm(sdUh + k0, LDG), dl = frag_rm(sdUl + k0, LDG);
            dS[j] = mfma(qh, gh, dS[j]);
            d2 = mfma(wa, dh, d2);
            dS[j] = mfma(qh, gl, dS[j]);
            d2 = mfma(wa, dl, d2);
            dS[j] = mfma(ql, gh, dS[j]);
            d2 = mfma(wal, dh, d2);
          }
#pragma unroll
          for (int i = 0; i < 16; ++i) dS[j][i] += d2[i];
        }
      }
      __syncthreads();
    }
  }
  if (a.ds0) {
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int rt = w + 4 * j;
      if (rt < NRT) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
          a.ds0[((long)unit * K + rt * 32 + acc_row(i)) * V + v0 + acc_col()] = dS[j][i];
      }
    }
  }
}

// ===========================================================================
// gdn_bwd_state for K <= 128 with 8 wavefronts (reverse walk over chunks).  Waves 0-3 compute and
// load nothing inside the walk; waves 4-7 move memory.  Per chunk c (dS' = gradient of the state
// after chunk c):
//   phase A  compute: dU = P^T dO + fac (K dS') (16x16 tiles), dU rows to HBM, -dU^T (hi/lo) to LDS;
//                     then the dS' snapshot to HBM and scale gamma dO (hi/lo) to LDS
//            memory:  Qc, w, wl of c to LDS (row-major); loads of Qc, w, wl of c-1
//   phase B  compute: dS <- gamma_L dS' + Qc^T (scale gamma dO) - w^T dU (Qc^T, w^T and the dO
//                     operand by transposing LDS reads), dS^T (hi/lo) to LDS for chunk c-1
//            memory:  P^T, dO, k, fac of c-1 to LDS; loads of P^T, dO, k, g of c-2
// ===========================================================================
// Q32: the cleaned query arrives in fp32 (else bf16); a template parameter, so the memory loop has
// a single path.
// SD: the state-gradient snapshots leave as int16 rows with row scales (else hi/lo pairs)
template <int K, bool Q32, bool SD>
__global__ __launch_bounds__(kWalk8) void gdn_bwd_state_v3_kernel(const GdnArgs a, const int V) {
  constexpr int VB = 32, LDK = K + 16, LDP = BT + 16, LDO = VB + 16;
  constexpr int NM = 256;
  constexpr int RW = K / 4, NR16 = RW / 16;
  __shared__ __attribute__((aligned(16))) bf16 sPh[BT * LDP];   // P^T [r][t], hi
  __shared__ __attribute__((aligned(16))) bf16 sPl[BT * LDP];
  __shared__ __attribute__((aligned(16))) bf16 sdO[BT * LDO];   // dO [t][v]
  __shared__ __attribute__((aligned(16))) bf16 sgOh[BT * LDO];  // scale gamma_t dO [t][v], hi
  __shared__ __attribute__((aligned(16))) bf16 sgOl[BT * LDO];
  __shared__ __attribute__((aligned(16))) bf16 sK[BT * LDK];    // k [t][k]
  __shared__ __attribute__((aligned(16))) bf16 sdSh[VB * LDK];  // dS'^T [v][k], hi
  __shared__ __attribute__((aligned(16))) bf16 sdSl[VB * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sdUh[VB * LDP];  // -dU^T [v][t], hi
  __shared__ __attribute__((aligned(16))) bf16 sdUl[VB * LDP];
  __shared__ __attribute__((aligned(16))) bf16 sQh[BT * LDK];   // Qc [t][k], hi
  __shared__ __attribute__((aligned(16))) bf16 sQl[BT * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sW[BT * LDK];    // w [t][k]
  __shared__ __attribute__((aligned(16))) bf16 sWl[BT * LDK];
  __shared__ __attribute__((aligned(16))) float sFac[BT];    // exp(g_L - g_t), 0 beyond the chunk
  __shared__ __attribute__((aligned(16))) float sGam[BT];    // scale exp(g_t), 0 beyond the chunk
  __shared__ float sGL[1];

  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(wave_id()), l = lane_id();
  const bool mem = w >= 4;
  const int lm = tid - NM;
  const int nv = V / VB;
  int unit, vt;
  xcd_map(blockIdx.x, nv, a.N * a.H, unit, vt);
  const int n = unit / a.H, h = unit % a.H;
  long bos;
  int len;
  seq_bounds(a.cu, n, a.T, bos, len);
  const int nc = (len + BT - 1) / BT;
  const int gc0 = a.cu ? a.chunk_off[n] : n * a.NT;
  const int v0 = vt * VB;
  const long rsk = (long)a.H * K, rsv = (long)a.H * V;
  auto chunk_len = [&](int c) { return min(BT, len - c * BT); };
  auto tok_of = [&](int c) { return bos + (long)c * BT; };

  if (mem) {
    // operands of phase B (Qc, w, wl: chunk c) and of phase A (P^T, dO, k, g: chunk c-1)
    RowsF32<K, BT, NM> pq;
    RowsBf16<K, BT, NM> pw, pwl, pk;
    RowsF32<BT, BT, NM> pp;
    RowsBf16<VB, BT, NM> po;
    float pgt = 0.f;  // g of token lm % 64
    auto load_b = [&](int c) {
      const long tok0 = tok_of(c);
      const int L = chunk_len(c);
      if constexpr (Q32)
        pq.load(a.qc32 + (tok0 * a.H + h) * K, rsk, L, lm);
      else
        pq.load(nullptr, (const bf16*)a.qc16 + (tok0 * a.H + h) * K, rsk, L, lm);
      pw.load((const bf16*)a.w + (tok0 * a.H + h) * K, rsk, L, lm);
      pwl.load((const bf16*)a.wl + (tok0 * a.H + h) * K, rsk, L, lm);
    };
    auto load_a = [&](int c) {
      const long tok0 = tok_of(c);
      const int L = chunk_len(c);
      pp.load(a.PT + ((long)(gc0 + c) * a.H + h) * (BT * BT), BT, BT, lm);
      po.load((const bf16*)a.dout + (tok0 * a.H + h) * (long)V + v0, rsv, L, lm);
      pk.load((const bf16*)a.k + (tok0 * a.H + h) * K, rsk, L, lm);
      pgt = a.gcum[(tok0 + min(lm & (BT - 1), L - 1)) * a.H + h];
    };
    // phase-A tiles of chunk c: P^T (hi/lo), dO, k; fac, gamma (lane t of wave 4)
    auto stage_a = [&](int c) {
      const int L = chunk_len(c);
      pp.store_split(sPh, sPl, LDP, BT, lm);
      po.store(sdO, LDO, L, lm);
      pk.store(sK, LDK, L, lm);
      const float pgl = __shfl(pgt, L - 1);
      const float fac = l < L ? __expf(pgl - pgt) : 0.f;
      const float gam = l < L ? a.scale * __expf(pgt) : 0.f;
      if (w == 4) {
        sFac[l] = fac;
        sGam[l] = gam;
        if (l == 0) sGL[0] = __expf(pgl);
      }
    };
    // phase-B tiles of chunk c: Qc (hi/lo), w, wl
    auto stage_b = [&](int c) {
      const int L = chunk_len(c);
      pq.store_split(sQh, sQl, LDK, L, lm);
      pw.store(sW, LDK, L, lm);
      pwl.store(sWl, LDK, L, lm);
    };
    // Loads run one chunk ahead of their stage and are unconditional (chunk 0 again past the
    // start), so every pass issues the same memory operations.
    const int cl = nc - 1;
    if (nc > 0) {
      load_a(cl);
      load_b(cl);
      stage_a(cl);
      load_a(max(cl - 1, 0));
    }
    __syncthreads();
    for (int c = cl; c >= 0; --c) {
      // ---- phase A: phase-B tiles of c; loads of Qc, w, wl of c-1
      stage_b(c);
      load_b(max(c - 1, 0));
      __syncthreads();
      // ---- phase B: phase-A tiles of c-1; loads of P^T, dO, k, g of c-2
      stage_a(max(c - 1, 0));
      load_a(max(c - 2, 0));
      __syncthreads();
    }
    return;
  }

  // compute waves: dS rows [RW w, RW w + RW) x 32 value columns as 16x16 tiles
  f32x4 dS[NR16][2];
#pragma unroll
  for (int rt = 0; rt < NR16; ++rt)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      dS[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (a.ds_fin) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          dS[rt][ct][i] = a.ds_fin[((long)unit * K + RW * w + 16 * rt + 4 * (l >> 4) + i) * V + v0 + 16 * ct + (l & 15)];
      }
    }
#pragma unroll
  for (int rt = 0; rt < NR16; ++rt)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) acc16_to_lds_t(dS[rt][ct], sdSh + 16 * ct * LDK, sdSl + 16 * ct * LDK, LDK, RW * w + 16 * rt);
  __syncthreads();
  for (int c = nc - 1; c >= 0; --c) {
    const int L = chunk_len(c);
    const long tok0 = tok_of(c);
    // ---- phase A: dU rows [16 w, 16 w + 16) = P^T dO + fac (K dS')
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    f32x4 acc2[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int k0 = 0; k0 < BT; k0 += 32) {
      const bf16x8 ph = frag16_rm(sPh + 16 * w * LDP + k0, LDP), pl = frag16_rm(sPl + 16 * w * LDP + k0, LDP);
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        const bf16x8 o = frag16_tr(sdO + k0 * LDO + 16 * ct, LDO);
        acc[ct] = mfma16(ph, o, acc[ct]);
        acc[ct] = mfma16(pl, o, acc[ct]);
      }
    }
#pragma unroll
    for (int k0 = 0; k0 < K; k0 += 32) {
      const bf16x8 kf = frag16_rm(sK + 16 * w * LDK + k0, LDK);
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        acc2[ct] = mfma16(kf, frag16_rm(sdSh + 16 * ct * LDK + k0, LDK), acc2[ct]);
        acc2[ct] = mfma16(kf, frag16_rm(sdSl + 16 * ct * LDK + k0, LDK), acc2[ct]);
      }
    }
    const float gL = sGL[0];
    const int rb = 16 * w + 4 * (l >> 4);
    const f32x4 fac = *(const f32x4*)(sFac + rb);
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const int cc = 16 * ct + (l & 15);
      f32x4 du, ndu;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        du[i] = rb + i < L ? acc[ct][i] + fac[i] * acc2[ct][i] : 0.f;
        ndu[i] = -du[i];
      }
      auto dug = gmem(a.dU) + (tok0 + rb) * rsv + (long)h * V + v0 + cc;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (rb + i < L) dug[i * rsv] = du[i];
      acc16_to_lds_t(ndu, sdUh + 16 * ct * LDP, sdUl + 16 * ct * LDP, LDP, 16 * w);
    }
    // with the products done: the dS' snapshot (hi/lo [v][k] rows, 16-byte pieces) to HBM, and scale
    // gamma dO (hi/lo) of chunk c for phase B (the memory waves are the longer path in this phase)
    {
      constexpr int VPR = K / 8;
      const int gc = gc0 + c;
      if constexpr (SD) {
#pragma unroll
        for (int j = 0; j < (VB * VPR) / NM; ++j) {
          const int idx = tid + j * NM, r = idx / VPR, cc = (idx % VPR) * 8;
          const long row = ((long)gc * a.H + h) * V + v0 + r;
          snap16_store<K>(sdSh + r * LDK + cc, sdSl + r * LDK + cc, (short*)a.dhT + row * K + cc, (float*)a.dhTl + row, tid);
        }
      } else {
#pragma unroll
        for (int j = 0; j < (2 * VB * VPR) / NM; ++j) {
          const int idx = tid + j * NM;
          const int which = idx / (VB * VPR), e = idx % (VB * VPR);
          const int r = e / VPR, cc = (e % VPR) * 8;
          const bf16* src = which ? sdSl : sdSh;
          bf16* dst = which ? (bf16*)a.dhTl : (bf16*)a.dhT;
          *gmem((bf16x8*)(dst + (((long)gc * a.H + h) * V + v0 + r) * K + cc)) = *(const bf16x8*)(src + r * LDK + cc);
        }
      }
      const int r = tid / (VB / 8), cc = (tid % (VB / 8)) * 8;
      const float sc = sGam[r];
      const bf16x8 o = *(const bf16x8*)(sdO + r * LDO + cc);
      bf16x8 vh, vl;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        bf16 x, y;
        split2(sc * (float)o[i], x, y);
        vh[i] = x;
        vl[i] = y;
      }
      *(bf16x8*)(sgOh + r * LDO + cc) = vh;
      *(bf16x8*)(sgOl + r * LDO + cc) = vl;
    }
    __syncthreads();

    // ---- phase B: dS <- gamma_L dS' + Qc^T (scale gamma dO) - w^T dU
#pragma unroll
    for (int rt = 0; rt < NR16; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) dS[rt][ct] *= gL;
#pragma unroll
    for (int k0 = 0; k0 < BT; k0 += 32) {
      bf16x8 gh[2], gl[2], dh[2], dl[2];
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        gh[ct] = frag16_tr(sgOh + k0 * LDO + 16 * ct, LDO);
        gl[ct] = frag16_tr(sgOl + k0 * LDO + 16 * ct, LDO);
        dh[ct] = frag16_rm(sdUh + 16 * ct * LDP + k0, LDP);
        dl[ct] = frag16_rm(sdUl + 16 * ct * LDP + k0, LDP);
      }
#pragma unroll
      for (int rt = 0; rt < NR16; ++rt) {
        const int m0 = RW * w + 16 * rt;
        const bf16x8 qh = frag16_tr(sQh + k0 * LDK + m0, LDK), ql = frag16_tr(sQl + k0 * LDK + m0, LDK);
        const bf16x8 wh = frag16_tr(sW + k0 * LDK + m0, LDK), wl = frag16_tr(sWl + k0 * LDK + m0, LDK);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
          dS[rt][ct] = mfma16(qh, gh[ct], dS[rt][ct]);
          dS[rt][ct] = mfma16(qh, gl[ct], dS[rt][ct]);
          dS[rt][ct] = mfma16(ql, gh[ct], dS[rt][ct]);
          dS[rt][ct] = mfma16(wh, dh[ct], dS[rt][ct]);
          dS[rt][ct] = mfma16(wh, dl[ct], dS[rt][ct]);
          dS[rt][ct] = mfma16(wl, dh[ct], dS[rt][ct]);
        }
      }
    }
#pragma unroll
    for (int rt = 0; rt < NR16; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
        acc16_to_lds_t(dS[rt][ct], sdSh + 16 * ct * LDK, sdSl + 16 * ct * LDK, LDK, RW * w + 16 * rt);
    __syncthreads();
  }
  if (a.ds0) {
#pragma unroll
    for (int rt = 0; rt < NR16; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          a.ds0[((long)unit * K + RW * w + 16 * rt + 4 * (l >> 4) + i) * V + v0 + 16 * ct + (l & 15)] = dS[rt][ct][i];
  }
}

// ===========================================================================
// gdn_bwd_dqkw: grid (K/64) * NTG * H, XCD-mapped (key-column block, chunk, head)
//   dQi = dO h^T, dKs = U dS'^T, dw = -dU h^T, dP = dO U^T   (contractions over V)
//   dq = scale gamma dQi + dPs K,  dk = fac dKs + dPs^T Qc,  dPs = dP o scale Gamma (causal)
//   dG partials: decay terms of O, P and the state update
// Every operand is staged once in the form its MFMA reads: the state tiles h^T, dS'^T arrive as [v][k] rows and are stored [k][v]
// from four-row patches; U, dU are stored as hi/lo rows; the post phase stores dPs^T, Qc^T, K^T
// (hi/lo where fp32) and does its row / column reductions over LDS with all threads.
// ===========================================================================
template <int K, bool SH, bool SD>
__global__ __launch_bounds__(kThreads) void gdn_bwd_dqkw_v2_kernel(const GdnArgs a, const int V) {
  constexpr int LDB = 64 + 8, LDE = 64 + 4, TILE = 64 * LDB;
  constexpr long kLoop = 9L * TILE * 2;
  constexpr long kPost = 5L * TILE * 2 + 2L * 64 * LDE * 4;
  constexpr long kBytes = kLoop > kPost ? kLoop : kPost;
  __shared__ __attribute__((aligned(16))) char region[kBytes];
  __shared__ __attribute__((aligned(16))) float sG[BT], sGam[BT], sFac[BT], sDG[BT], sTerm[BT], sMisc[8];
  // loop views
  bf16* sHk = (bf16*)region;  // h^T tile as [k][v]
  bf16* sHkl = sHk + TILE;
  bf16* sDk = sHkl + TILE;     // dS'^T tile as [k][v]
  bf16* sDkl = sDk + TILE;
  bf16* sdO = sDkl + TILE;     // dO [t][v]
  bf16* sUh = sdO + TILE;      // U [t][v]
  bf16* sUl = sUh + TILE;
  bf16* sdUh = sUl + TILE;     // dU [t][v]
  bf16* sdUl = sdUh + TILE;
  // post views (same region)
  bf16* sPh = (bf16*)region;   // dPs^T [s][t]
  bf16* sPl = sPh + TILE;
  bf16* sQh = sPl + TILE;      // Qc^T [k][t]
  bf16* sQl = sQh + TILE;
  bf16* sKt = sQl + TILE;      // K^T [k][t]
  float* sE = (float*)(sKt + TILE);  // [64][LDE] products for row / column sums
  float* sPT = sE + 64 * LDE;        // P^T [s][t] (kt == 0)

  const int tid = threadIdx.x, w = wave_id(), l = lane_id();
  // the K / 64 key-column blocks of a (chunk, head) unit share the unit's dO, U, dU and P^T: they
  // run on one XCD (one L2) when the unit count allows it
  int unit, kt;
  xcd_map(blockIdx.x, K / 64, a.NTG * a.H, unit, kt);
  const int gc = unit / a.H, h = unit % a.H;
  int n, c0, L;
  long bos;
  if (!chunk_info(a, gc, n, c0, bos, L)) return;
  const long tok0 = bos + c0;
  const long rsk = (long)a.H * K, rsv = (long)a.H * V;
  const int k0c = kt * 64;
  const int tr = (w >> 1) * 32, tc = (w & 1) * 32;
  const int pr = (w == 0) ? 0 : 32, pc = (w == 2) ? 32 : 0;
  f32x16 dQi = zero16(), dKs = zero16(), dW = zero16(), dP = zero16();
  float hds = 0.f;

  // the state (SH) and state-gradient (SD) snapshots: int16 rows with row scales, else hi/lo pairs
  PatchBf16<64, 64> pH, pD;
  PatchBf16<64, SH ? 4 : 64> pHl;
  PatchBf16<64, SD ? 4 : 64> pDl;
  float scH[PatchBf16<64, 64>::N][4], scD[PatchBf16<64, 64>::N][4];
  PrefetchBf16<64, 64> pO;
  PrefetchF32Split<64, 64> pU, pdU;
  PatchF32<64, 64> pQ;
  PatchBf16<64, 64> pK;
  PrefetchF32<BT, BT> pP;
  float pgl = 0.f, pgt = 0.f;
  auto issue_loop = [&](int v0) {
    const long so = (((long)gc * a.H + h) * V + v0) * K + k0c;
    pH.load((const bf16*)a.hT + so, K, 64, tid);
    pD.load((const bf16*)a.dhT + so, K, 64, tid);
    const long sb = ((long)gc * a.H + h) * V + v0;
    if constexpr (SH)
      pH.load_scales((const float*)a.hTl + sb, 64, tid, scH);
    else
      pHl.load((const bf16*)a.hTl + so, K, 64, tid);
    if constexpr (SD)
      pD.load_scales((const float*)a.dhTl + sb, 64, tid, scD);
    else
      pDl.load((const bf16*)a.dhTl + so, K, 64, tid);
    pO.load((const bf16*)a.dout + (tok0 * a.H + h) * (long)V + v0, rsv, L);
    pU.load(a.U + (tok0 * a.H + h) * (long)V + v0, rsv, tid, L);
    pdU.load(a.dU + (tok0 * a.H + h) * (long)V + v0, rsv, tid, L);
  };
  auto issue_post = [&]() {
    pQ.load(a.qc32 ? a.qc32 + (tok0 * a.H + h) * K + k0c : nullptr,
            a.qc16 ? (const bf16*)a.qc16 + (tok0 * a.H + h) * K + k0c : nullptr, rsk, L, tid);
    pK.load((const bf16*)a.k + (tok0 * a.H + h) * K + k0c, rsk, L, tid);
    if (kt == 0) pP.load(a.PT + ((long)gc * a.H + h) * (BT * BT), BT, BT);
    if (tid < BT) {
      pgl = a.gcum[(tok0 + L - 1) * a.H + h];
      pgt = (tid < L) ? a.gcum[(tok0 + tid) * a.H + h] : pgl;
    }
  };
  issue_loop(0);

  for (int v0 = 0; v0 < V; v0 += 64) {
    if constexpr (SH) {
      pH.store_t_s16(sHk, sHkl, LDB, scH, tid);
    } else {
      pH.store_t(sHk, LDB, 64, tid);
      pHl.store_t(sHkl, LDB, 64, tid);
    }
    if constexpr (SD) {
      pD.store_t_s16(sDk, sDkl, LDB, scD, tid);
    } else {
      pD.store_t(sDk, LDB, 64, tid);
      pDl.store_t(sDkl, LDB, 64, tid);
    }
    pO.store(sdO, LDB, nullptr, 0);
    pU.store(sUh, sUl, LDB, tid, L);
    pdU.store(sdUh, sdUl, LDB, tid, L);
    __syncthreads();
    if (v0 + 64 < V) issue_loop(v0 + 64);
    else issue_post();
    {
      // <h, dS'> over the tile: row k = tid / 4, sixteen v per thread
      const int kk = tid >> 2, vs = (tid & 3) * 16;
#pragma unroll
      for (int q = 0; q < 16; q += 8) {
        const int e = kk * LDB + vs + q;
        const bf16x8 x1 = *(const bf16x8*)(sHk + e), x2 = *(const bf16x8*)(sHkl + e);
        const bf16x8 y1 = *(const bf16x8*)(sDk + e), y2 = *(const bf16x8*)(sDkl + e);
#pragma unroll
        for (int i = 0; i < 8; ++i) hds += ((float)x1[i] + (float)x2[i]) * ((float)y1[i] + (float)y2[i]);
      }
    }
#pragma unroll
    for (int k0 = 0; k0 < 64; k0 += 16) {
      const bf16x8 oa = frag_rm(sdO + tr * LDB + k0, LDB);
      const bf16x8 hb = frag_rm(sHk + tc * LDB + k0, LDB), hbl = frag_rm(sHkl + tc * LDB + k0, LDB);
      dQi = mfma(oa, hb, dQi);
      dQi = mfma(oa, hbl, dQi);
      const bf16x8 uh = frag_rm(sUh + tr * LDB + k0, LDB), ul = frag_rm(sUl + tr * LDB + k0, LDB);
      const bf16x8 db = frag_rm(sDk + tc * LDB + k0, LDB), dbl = frag_rm(sDkl + tc * LDB + k0, LDB);
      dKs = mfma(uh, db, dKs);
      dKs = mfma(ul, db, dKs);
      dKs = mfma(uh, dbl, dKs);
      const bf16x8 dh = frag_rm(sdUh + tr * LDB + k0, LDB), dl = frag_rm(sdUl + tr * LDB + k0, LDB);
      dW = mfma(dh, hb, dW);
      dW = mfma(dl, hb, dW);
      dW = mfma(dh, hbl, dW);
      if (w < 3) {
        const bf16x8 pa = frag_rm(sdO + pr * LDB + k0, LDB);
        dP = mfma(pa, frag_rm(sUh + pc * LDB + k0, LDB), dP);
        dP = mfma(pa, frag_rm(sUl + pc * LDB + k0, LDB), dP);
      }
    }
    __syncthreads();
  }
  hds = group_sum(hds, 64);
  if (l == 0) sMisc[w] = hds;

  // ---- post stage (the loop ended with a barrier; its tiles are dead)
  pQ.store_t(sQh, sQl, LDB, L, tid);
  pK.store_t(sKt, LDB, L, tid);
  if (kt == 0) {
#pragma unroll
    for (int j = 0; j < PrefetchF32<BT, BT>::N; ++j) {
      const int idx = tid + j * kThreads;
      if (idx < BT * (BT / 4)) *(f32x4*)(sPT + (idx / (BT / 4)) * LDE + (idx % (BT / 4)) * 4) = pP.v[j];
    }
  }
  if (tid < BT) {
    sG[tid] = pgt;
    sGam[tid] = __expf(pgt);
    sFac[tid] = __expf(pgl - pgt);
    if (tid == 0) sMisc[4] = __expf(pgl);
  }
  __syncthreads();

  // ---- dP: mask, decay terms of P (kt == 0), dPs^T as hi/lo
  {
    f32x16 ps;
    if (w < 3) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = pr + acc_row(i), c = pc + acc_col();
        const bool keep = r >= c;
        dP[i] = keep ? dP[i] : 0.f;
        ps[i] = keep ? dP[i] * a.scale * __expf(sG[r] - sG[c]) : 0.f;
      }
      if (kt == 0) {
        const int c = pc + acc_col();
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int i4 = pr + acc_row(4 * g);
          const f32x4 pv = *(const f32x4*)(sPT + c * LDE + i4);  // P[i][c] = P^T[c][i]
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) sE[(i4 + ii) * LDE + c] = dP[4 * g + ii] * pv[ii];
        }
      }
      acc_to_lds_t(ps, sPh + pc * LDB, sPl + pc * LDB, LDB, pr);
    } else {
      if (kt == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) sE[acc_row(i) * LDE + 32 + acc_col()] = 0.f;
      }
      acc_to_lds_t(zero16(), sPh + 32 * LDB, sPl + 32 * LDB, LDB, 0);
    }
  }
  __syncthreads();
  if (tid < 64) {
    float s = 0.f;
    if (kt == 0) {
#pragma unroll
      for (int q = 0; q < 64; q += 4) {
        const f32x4 x = *(const f32x4*)(sE + tid * LDE + q);
        s += x[0] + x[1] + x[2] + x[3];
      }
    }
    sDG[tid] = s;
  } else if (tid < 128) {
    float s = 0.f;
    if (kt == 0) {
#pragma unroll 8
      for (int i = 0; i < 64; ++i) s += sE[i * LDE + tid - 64];
    }
    sTerm[tid - 64] = s;
  }
  __syncthreads();

  // ---- dq tile = scale gamma dQi + dPs K[:, tile]; decay term of O: dG_i += sum_k dQi_ik qc_ik
  {
    const int c = tc + acc_col();
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int i4 = tr + acc_row(4 * g);
      const f32x4 gm = *(const f32x4*)(sGam + i4);
      const bf16x4 qh4 = *(const bf16x4*)(sQh + c * LDB + i4), ql4 = *(const bf16x4*)(sQl + c * LDB + i4);
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int k = 4 * g + ii;
        dQi[k] *= a.scale * gm[ii];
        sE[(i4 + ii) * LDE + c] = dQi[k] * ((float)qh4[ii] + (float)ql4[ii]);
      }
    }
#pragma unroll
    for (int k0 = 0; k0 < BT; k0 += 16) {
      const bf16x8 kb = frag_rm(sKt + tc * LDB + k0, LDB);
      dQi = mfma(frag32_tr(sPh + k0 * LDB + tr, LDB), kb, dQi);
      dQi = mfma(frag32_tr(sPl + k0 * LDB + tr, LDB), kb, dQi);
    }
    const int r0 = tr + acc_row(0);
    float* dq = a.dq32 + (tok0 + r0) * rsk + (long)h * K + k0c + c;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (r0 + acc_drow(i) < L) dq[acc_drow(i) * rsk] = dQi[i];
  }
  __syncthreads();
  if (tid < 64) {
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < 64; q += 4) {
      const f32x4 x = *(const f32x4*)(sE + tid * LDE + q);
      s += x[0] + x[1] + x[2] + x[3];
    }
    sDG[tid] = sDG[tid] - sTerm[tid] + s;
  }
  __syncthreads();

  // ---- dk tile = fac dKs + dPs^T Qc[:, tile];  state-update decay term_j = sum_k fac dKs_jk k_jk
  {
    const int c = tc + acc_col();
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int i4 = tr + acc_row(4 * g);
      const f32x4 fc = *(const f32x4*)(sFac + i4);
      const bf16x4 k4 = *(const bf16x4*)(sKt + c * LDB + i4);
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int k = 4 * g + ii;
        dKs[k] *= fc[ii];
        sE[(i4 + ii) * LDE + c] = dKs[k] * (float)k4[ii];
      }
    }
#pragma unroll
    for (int k0 = 0; k0 < BT; k0 += 16) {
      const bf16x8 ah = frag_rm(sPh + tr * LDB + k0, LDB), al = frag_rm(sPl + tr * LDB + k0, LDB);
      const bf16x8 bh = frag_rm(sQh + tc * LDB + k0, LDB);
      dKs = mfma(ah, bh, dKs);
      dKs = mfma(ah, frag_rm(sQl + tc * LDB + k0, LDB), dKs);
      dKs = mfma(al, bh, dKs);
    }
    const int r0 = tr + acc_row(0);
    const long gi = (tok0 + r0) * rsk + (long)h * K + k0c + c;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (r0 + acc_drow(i) < L) {
        a.dkp32[gi + acc_drow(i) * rsk] = dKs[i];
        a.dw32[gi + acc_drow(i) * rsk] = -dW[i];
      }
    }
  }
  __syncthreads();
  if (tid < 64) {
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < 64; q += 4) {
      const f32x4 x = *(const f32x4*)(sE + tid * LDE + q);
      s += x[0] + x[1] + x[2] + x[3];
    }
    sTerm[tid] = s;  // term_j
  }
  __syncthreads();
  if (tid < L) {
    float d = sDG[tid] - sTerm[tid];
    if (tid == L - 1) {
      float tot = 0.f;
      for (int j = 0; j < L; ++j) tot += sTerm[j];
      d += tot + sMisc[4] * (sMisc[0] + sMisc[1] + sMisc[2] + sMisc[3]);
    }
    const long ntok = a.cu ? (long)a.cu[a.N] : (long)a.N * a.T;
    a.dgp[(long)kt * ntok * a.H + (tok0 + tid) * a.H + h] = d;
  }
}

// ===========================================================================
// gdn_bwd_dqkw for K = 128 on 8 waves: one workgroup per (chunk, head) instead of one per 64-column
// key tile.  Waves 0-3 (group 0) and 4-7 (group 1) each run the per-tile computation of
// gdn_bwd_dqkw_v2_kernel for key columns [64 g, 64 g + 64); the value-side tiles (dO, U, dU), the
// product dP = dO U^T with its masked, decayed form dPs and the decay terms of P are staged or
// computed once and shared.  Each group writes its own decay-gradient partial.
// ===========================================================================
template <int K>
__global__ __launch_bounds__(kWalk8) void gdn_bwd_dqkw_v3_kernel(const GdnArgs a, const int V) {
  static_assert(K == 128, "two key tiles of 64");
  constexpr int LDB = 64 + 8, LDE = 64 + 4, TILE = 64 * LDB, NG = 2;
  constexpr long kLoop = (4L * NG + 5) * TILE * 2;
  constexpr long kPost = (2L + 3 * NG) * TILE * 2 + (NG + 1L) * 64 * LDE * 4;
  constexpr long kBytes = kLoop > kPost ? kLoop : kPost;
  __shared__ __attribute__((aligned(16))) char region[kBytes];
  __shared__ __attribute__((aligned(16))) float sG[BT], sGam[BT], sFac[BT];
  __shared__ __attribute__((aligned(16))) float sDG[NG][BT], sTerm[NG][BT], sMisc[NG][8];

  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(wave_id()), l = lane_id();
  const int g = w >> 2, gw = w & 3, gt = tid & 255;  // group (key tile), wave and thread in the group
  const int gc = blockIdx.y, h = blockIdx.z;
  int n, c0, L;
  long bos;
  if (!chunk_info(a, gc, n, c0, bos, L)) return;
  const long tok0 = bos + c0;
  const long rsk = (long)a.H * K, rsv = (long)a.H * V;
  const int k0c = g * 64;
  // loop views: shared value-side tiles, then four state tiles per group
  bf16* sdO = (bf16*)region;   // dO [t][v]
  bf16* sUh = sdO + TILE;      // U [t][v]
  bf16* sUl = sUh + TILE;
  bf16* sdUh = sUl + TILE;     // dU [t][v]
  bf16* sdUl = sdUh + TILE;
  bf16* sHk = sdUl + TILE + g * 4 * TILE;  // h^T tile as [k][v]
  bf16* sHkl = sHk + TILE;
  bf16* sDk = sHkl + TILE;                 // dS'^T tile as [k][v]
  bf16* sDkl = sDk + TILE;
  // post views (same region)
  bf16* sPh = (bf16*)region;   // dPs^T [s][t] (shared)
  bf16* sPl = sPh + TILE;
  bf16* sQh = sPl + TILE + g * 3 * TILE;  // Qc^T [k][t] of this group's columns
  bf16* sQl = sQh + TILE;
  bf16* sKt = sQl + TILE;                 // K^T [k][t]
  float* sEall = (float*)(region + (2L + 3 * NG) * TILE * 2);
  float* sE = sEall + g * 64 * LDE;       // [64][LDE] products for row / column sums
  float* sPT = sEall + NG * 64 * LDE;     // P^T [s][t]

  const int tr = (gw >> 1) * 32, tc = (gw & 1) * 32;
  const int pr = (gw == 0) ? 0 : 32, pc = (gw == 2) ? 32 : 0;
  f32x16 dQi = zero16(), dKs = zero16(), dW = zero16(), dP = zero16();
  float hds = 0.f;

  PatchBf16<64, 64> pH, pHl, pD, pDl;
  RowsBf16<64, 64, 256> pO;
  PrefetchF32Split<64, 64> pU;  // group 0: U, group 1: dU
  PatchF32<64, 64> pQ;
  PatchBf16<64, 64> pK;
  RowsF32<BT, BT, 256> pP;
  float pgl = 0.f, pgt = 0.f;
  auto issue_loop = [&](int v0) {
    const long so = (((long)gc * a.H + h) * V + v0) * K + k0c;
    pH.load((const bf16*)a.hT + so, K, 64, gt);
    pHl.load((const bf16*)a.hTl + so, K, 64, gt);
    pD.load((const bf16*)a.dhT + so, K, 64, gt);
    pDl.load((const bf16*)a.dhTl + so, K, 64, gt);
    if (g == 0) {
      pO.load((const bf16*)a.dout + (tok0 * a.H + h) * (long)V + v0, rsv, L, gt);
      pU.load(a.U + (tok0 * a.H + h) * (long)V + v0, rsv, gt, L);
    } else {
      pU.load(a.dU + (tok0 * a.H + h) * (long)V + v0, rsv, gt, L);
    }
  };
  auto issue_post = [&]() {
    pQ.load(a.qc32 ? a.qc32 + (tok0 * a.H + h) * K + k0c : nullptr,
            a.qc16 ? (const bf16*)a.qc16 + (tok0 * a.H + h) * K + k0c : nullptr, rsk, L, gt);
    pK.load((const bf16*)a.k + (tok0 * a.H + h) * K + k0c, rsk, L, gt);
    if (g == 0) {
      pP.load(a.PT + ((long)gc * a.H + h) * (BT * BT), BT, BT, gt);
      if (gt < BT) {
        pgl = a.gcum[(tok0 + L - 1) * a.H + h];
        pgt = a.gcum[(tok0 + min(gt, L - 1)) * a.H + h];
      }
    }
  };
  issue_loop(0);

  for (int v0 = 0; v0 < V; v0 += 64) {
    pH.store_t(sHk, LDB, 64, gt);
    pHl.store_t(sHkl, LDB, 64, gt);
    pD.store_t(sDk, LDB, 64, gt);
    pDl.store_t(sDkl, LDB, 64, gt);
    if (g == 0) {
      pO.store(sdO, LDB, L, gt);
      pU.store(sUh, sUl, LDB, gt, L);
    } else {
      pU.store(sdUh, sdUl, LDB, gt, L);
    }
    __syncthreads();
    if (v0 + 64 < V) issue_loop(v0 + 64);
    {
      // <h, dS'> over the tile: row k = gt / 4, sixteen v per thread
      const int kk = gt >> 2, vs = (gt & 3) * 16;
#pragma unroll
      for (int q = 0; q < 16; q += 8) {
        const int e = kk * LDB + vs + q;
        const bf16x8 x1 = *(const bf16x8*)(sHk + e), x2 = *(const bf16x8*)(sHkl + e);
        const bf16x8 y1 = *(const bf16x8*)(sDk + e), y2 = *(const bf16x8*)(sDkl + e);
#pragma unroll
        for (int i = 0; i < 8; ++i) hds += ((float)x1[i] + (float)x2[i]) * ((float)y1[i] + (float)y2[i]);
      }
    }
#pragma unroll
    for (int k0 = 0; k0 < 64; k0 += 16) {
      const bf16x8 oa = frag_rm(sdO + tr * LDB + k0, LDB);
      const bf16x8 hb = frag_rm(sHk + tc * LDB + k0, LDB), hbl = frag_rm(sHkl + tc * LDB + k0, LDB);
      dQi = mfma(oa, hb, dQi);
      dQi = mfma(oa, hbl, dQi);
      const bf16x8 uh = frag_rm(sUh + tr * LDB + k0, LDB), ul = frag_rm(sUl + tr * LDB + k0, LDB);
      const bf16x8 db = frag_rm(sDk + tc * LDB + k0, LDB), dbl = frag_rm(sDkl + tc * LDB + k0, LDB);
      dKs = mfma(uh, db, dKs);
      dKs = mfma(ul, db, dKs);
      dKs = mfma(uh, dbl, dKs);
      const bf16x8 dh = frag_rm(sdUh + tr * LDB + k0, LDB), dl = frag_rm(sdUl + tr * LDB + k0, LDB);
      dW = mfma(dh, hb, dW);
      dW = mfma(dl, hb, dW);
      dW = mfma(dh, hbl, dW);
      if (g == 0 && gw < 3) {
        const bf16x8 pa = frag_rm(sdO + pr * LDB + k0, LDB);
        dP = mfma(pa, frag_rm(sUh + pc * LDB + k0, LDB), dP);
        dP = mfma(pa, frag_rm(sUl + pc * LDB + k0, LDB), dP);
      }
    }
    __syncthreads();
  }
  hds = group_sum(hds, 64);
  if (l == 0) sMisc[g][gw] = hds;

  // ---- post stage (the loop ended with a barrier; its tiles are dead).  Its operands are loaded
  // here rather than during the last value block: with two waves per SIMD the registers do not
  // hold both.
  issue_post();
  pQ.store_t(sQh, sQl, LDB, L, gt);
  pK.store_t(sKt, LDB, L, gt);
  if (g == 0) {
    pP.store(sPT, LDE, BT, gt);
    if (gt < BT) {
      sG[gt] = pgt;
      sGam[gt] = __expf(pgt);
      sFac[gt] = __expf(pgl - pgt);
      if (gt == 0) {
        sMisc[0][4] = __expf(pgl);
        sMisc[1][4] = __expf(pgl);
      }
    }
  }
  __syncthreads();

  // ---- dP (group 0): mask, decay terms of P, dPs^T as hi/lo
  if (g == 0) {
    f32x16 ps;
    if (gw < 3) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = pr + acc_row(i), c = pc + acc_col();
        const bool keep = r >= c;
        dP[i] = keep ? dP[i] : 0.f;
        ps[i] = keep ? dP[i] * a.scale * __expf(sG[r] - sG[c]) : 0.f;
      }
      const int c = pc + acc_col();
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int i4 = pr + acc_row(4 * q);
        const f32x4 pv = *(const f32x4*)(sPT + c * LDE + i4);  // P[i][c] = P^T[c][i]
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) sE[(i4 + ii) * LDE + c] = dP[4 * q + ii] * pv[ii];
      }
      acc_to_lds_t(ps, sPh + pc * LDB, sPl + pc * LDB, LDB, pr);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) sE[acc_row(i) * LDE + 32 + acc_col()] = 0.f;
      acc_to_lds_t(zero16(), sPh + 32 * LDB, sPl + 32 * LDB, LDB, 0);
    }
  }
  __syncthreads();
  if (gt < 64) {
    float s = 0.f;
    if (g == 0) {
#pragma unroll
      for (int q = 0; q < 64; q += 4) {
        const f32x4 x = *(const f32x4*)(sE + gt * LDE + q);
        s += x[0] + x[1] + x[2] + x[3];
      }
    }
    sDG[g][gt] = s;
  } else if (gt < 128) {
    float s = 0.f;
    if (g == 0) {
#pragma unroll 8
      for (int i = 0; i < 64; ++i) s += sE[i * LDE + gt - 64];
    }
    sTerm[g][gt - 64] = s;
  }
  __syncthreads();

  // ---- dq tile = scale gamma dQi + dPs K[:, tile]; decay term of O: dG_i += sum_k dQi_ik qc_ik
  {
    const int c = tc + acc_col();
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int i4 = tr + acc_row(4 * q);
      const f32x4 gm = *(const f32x4*)(sGam + i4);
      const bf16x4 qh4 = *(const bf16x4*)(sQh + c * LDB + i4), ql4 = *(const bf16x4*)(sQl + c * LDB + i4);
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int k = 4 * q + ii;
        dQi[k] *= a.scale * gm[ii];
        sE[(i4 + ii) * LDE + c] = dQi[k] * ((float)qh4[ii] + (float)ql4[ii]);
      }
    }
#pragma unroll
    for (int k0 = 0; k0 < BT; k0 += 16) {
      const bf16x8 kb = frag_rm(sKt + tc * LDB + k0, LDB);
      dQi = mfma(frag32_tr(sPh + k0 * LDB + tr, LDB), kb, dQi);
      dQi = mfma(frag32_tr(sPl + k0 * LDB + tr, LDB), kb, dQi);
    }
    const int r0 = tr + acc_row(0);
    float* dq = a.dq32 + (tok0 + r0) * rsk + (long)h * K + k0c + c;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (r0 + acc_drow(i) < L) dq[acc_drow(i) * rsk] = dQi[i];
  }
  __syncthreads();
  if (gt < 64) {
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < 64; q += 4) {
      const f32x4 x = *(const f32x4*)(sE + gt * LDE + q);
      s += x[0] + x[1] + x[2] + x[3];
    }
    sDG[g][gt] = sDG[g][gt] - sTerm[g][gt] + s;
  }
  __syncthreads();

  // ---- dk tile = fac dKs + dPs^T Qc[:, tile];  state-update decay term_j = sum_k fac dKs_jk k_jk
  {
    const int c = tc + acc_col();
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int i4 = tr + acc_row(4 * q);
      const f32x4 fc = *(const f32x4*)(sFac + i4);
      const bf16x4 k4 = *(const bf16x4*)(sKt + c * LDB + i4);
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int k = 4 * q + ii;
        dKs[k] *= fc[ii];
        sE[(i4 + ii) * LDE + c] = dKs[k] * (float)k4[ii];
      }
    }
#pragma unroll
    for (int k0 = 0; k0 < BT; k0 += 16) {
      const bf16x8 ah = frag_rm(sPh + tr * LDB + k0, LDB), al = frag_rm(sPl + tr * LDB + k0, LDB);
      const bf16x8 bh = frag_rm(sQh + tc * LDB + k0, LDB);
      dKs = mfma(ah, bh, dKs);
      dKs = mfma(ah, frag_rm(sQl + tc * LDB + k0, LDB), dKs);
      dKs = mfma(al, bh, dKs);
    }
    const int r0 = tr + acc_row(0);
    const long gi = (tok0 + r0) * rsk + (long)h * K + k0c + c;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (r0 + acc_drow(i) < L) {
        a.dkp32[gi + acc_drow(i) * rsk] = dKs[i];
        a.dw32[gi + acc_drow(i) * rsk] = -dW[i];
      }
    }
  }
  __syncthreads();
  if (gt < 64) {
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < 64; q += 4) {
      const f32x4 x = *(const f32x4*)(sE + gt * LDE + q);
      s += x[0] + x[1] + x[2] + x[3];
    }
    sTerm[g][gt] = s;  // term_j
  }
  __syncthreads();
  if (gt < L) {
    float d = sDG[g][gt] - sTerm[g][gt];
    if (gt == L - 1) {
      float tot = 0.f;
      for (int j = 0; j < L; ++j) tot += sTerm[g][j];
      d += tot + sMisc[g][4] * (sMisc[g][0] + sMisc[g][1] + sMisc[g][2] + sMisc[g][3]);
    }
    const long ntok = a.cu ? (long)a.cu[a.N] : (long)a.N * a.T;
    a.dgp[(long)g * ntok * a.H + (tok0 + gt) * a.H + h] = d;
  }
}

// ===========================================================================
// gdn_bwd_wy: grid (NTG, H)  -- backward through w = T diag(beta gamma) K, u = T diag(beta) V,
// T = (I + A)^-1, A = strict_lower(diag(beta) (K K^T o Gamma)), with every operand in the form its
// MFMA reads.  Products whose transpose is needed later are computed in the transposed orientation and
// written back transposed (acc_to_lds_t), so all fragments are 16-byte row reads:
//   phase 1  (dT K-part)^T, (dT V-part)^T over key / value tiles; K K^T
//   phase 2  M1 = dT T^T -> M1^T;  dA = -T^T M1 and dA^T = -M1^T T in registers
//   phase 3  dbeta / dG terms of A;  dAs = dA o beta_r Gamma_rc stored as rows and as columns
//   phase 4  per key tile: dk = dk_part + dAs K + dAs^T K + diag(beta gamma) T^T dw
//   phase 5  per value tile: dv = diag(beta) T^T dU;  dbeta += (T^T dU) . v
// Row / column reductions go through LDS and all threads.
// ===========================================================================
template <int K>
__global__ __launch_bounds__(kThreads) void gdn_bwd_wy_v2_kernel(const GdnArgs a, const int V) {
  constexpr int LDB = 64 + 8, LDE = 64 + 4, TILE = 64 * LDB, FT = 64 * LDE;
  constexpr long kScr1 = 4L * TILE * 2;                    // phases 1-2: sX hi/lo + sR, then dT, M1^T
  constexpr long kScr3 = 2L * FT * 4;                      // phase 3: two product tiles
  constexpr long kScr4 = 3L * TILE * 2 + 2L * FT * 4;      // phase 4: K^T, dw^T hi/lo, dk_part, products
  constexpr long kScr5 = 3L * TILE * 2 + 1L * FT * 4;      // phase 5: dU^T hi/lo, V, products
  constexpr long kScr = kScr1 > kScr3 ? (kScr1 > kScr4 ? kScr1 : kScr4) : (kScr3 > kScr4 ? kScr3 : kScr4);
  static_assert(kScr >= kScr5, "scratch");
  __shared__ __attribute__((aligned(16))) bf16 sTh[TILE], sTl[TILE];    // T [r][c]
  __shared__ __attribute__((aligned(16))) bf16 sTth[TILE], sTtl[TILE];  // T^T [r][c] = T[c][r]
  __shared__ __attribute__((aligned(16))) bf16 sAh[TILE], sAl[TILE];    // dAs [r][c]
  __shared__ __attribute__((aligned(16))) bf16 sATh[TILE], sATl[TILE];  // dAs^T [c][r]
  __shared__ __attribute__((aligned(16))) char scr[kScr];
  __shared__ __attribute__((aligned(16))) float sG[BT], sBeta[BT], sGam[BT], sDB[BT], sDG[BT], sRow[BT], sCol[BT];
  // phase 1 views
  bf16* sXh = (bf16*)scr;  // fp32 tile rows [t][c], hi
  bf16* sXl = sXh + TILE;
  bf16* sR = sXl + TILE;   // bf16 tile rows [t][c]
  // phase 2 views
  bf16* sDh = (bf16*)scr;  // dT [r][c]
  bf16* sDl = sDh + TILE;
  bf16* sMh = sDl + TILE;  // M1^T [c][r]
  bf16* sMl = sMh + TILE;
  // phase 3 views
  float* sE1 = (float*)scr;
  float* sE2 = sE1 + FT;
  // phase 4 / 5 views
  bf16* sCt = (bf16*)scr;  // K^T [k][t] (phase 4) / V [t][v] (phase 5)
  bf16* sFh = sCt + TILE;  // dw^T [k][t] (phase 4) / dU^T [v][t] (phase 5), hi
  bf16* sFl = sFh + TILE;
  float* sE = (float*)(sFl + TILE);  // products [t][c]
  float* sKp = sE + FT;              // dk_part [t][k] (phase 4)

  const int tid = threadIdx.x, w = wave_id();
  const int gc = blockIdx.x, h = blockIdx.y;
  int n, c0, L;
  long bos;
  if (!chunk_info(a, gc, n, c0, bos, L)) return;
  const long tok0 = bos + c0;
  const long rsk = (long)a.H * K, rsv = (long)a.H * V;
  const long ntok = a.cu ? (long)a.cu[a.N] : (long)a.N * a.T;
  const int nkt = K / 64, nv = V / 64;

  // jobs (one fp32 tile, one bf16 tile, one more fp32 tile in phase 4), one ahead in registers:
  // [0, nkt): dw, k   [nkt, nkt+nv): dU, v   [nkt+nv, 2nkt+nv): dw, k, dk_part   then dU, v
  const int nA = nkt, nB = nkt + nv, nC = 2 * nkt + nv, njobs = 2 * (nkt + nv);
  PatchF32<64, BT> pF, pF2;
  PatchBf16<64, BT> pB;
  auto issue = [&](int j) {
    const bool kside = j < nA || (j >= nB && j < nC);
    const int col = 64 * (j < nA ? j : j < nB ? j - nA : j < nC ? j - nB : j - nC);
    if (kside) {
      pF.load(a.dw32 + (tok0 * a.H + h) * K + col, nullptr, rsk, L, tid);
      pB.load((const bf16*)a.k + (tok0 * a.H + h) * K + col, rsk, L, tid);
      if (j >= nB) pF2.load(a.dkp32 + (tok0 * a.H + h) * K + col, nullptr, rsk, L, tid);
    } else {
      pF.load(a.dU + (tok0 * a.H + h) * (long)V + col, nullptr, rsv, L, tid);
      pB.load((const bf16*)a.v + (tok0 * a.H + h) * (long)V + col, rsv, L, tid);
    }
  };
  issue(0);
  {
    PatchF32<BT, BT> pT;
    pT.load(a.tmat + ((long)gc * a.H + h) * (BT * BT), nullptr, BT, BT, tid);
    if (tid < BT) {
      const float gl = a.gcum[(tok0 + L - 1) * a.H + h];
      const float gt = (tid < L) ? a.gcum[(tok0 + tid) * a.H + h] : gl;
      sG[tid] = gt;
      sGam[tid] = __expf(gt);
      sBeta[tid] = (tid < L) ? a.beta[(tok0 + tid) * a.H + h] : 0.f;
      float dg = 0.f;
      if (tid < L)
        for (int kt = 0; kt < nkt; ++kt) dg += a.dgp[(long)kt * ntok * a.H + (tok0 + tid) * a.H + h];
      sDG[tid] = dg;
      sDB[tid] = 0.f;
    }
    pT.store_rm(sTh, sTl, LDB, BT, tid);
    pT.store_t(sTth, sTtl, LDB, BT, tid);
  }
  int job = 0;
  const int R = blk_row3(w), C = blk_col3(w);  // lower 32 x 32 block of waves 0..2

  // ---- phase 1
  f32x16 dTk = zero16(), dTv = zero16(), kk = zero16();
  for (; job < nB; ++job) {
    pF.store_rm(sXh, sXl, LDB, L, tid);
    pB.store_rm(sR, LDB, L, tid);
    __syncthreads();
    if (job + 1 < njobs) issue(job + 1);
    if (w < 3) {
      const bool kside = job < nA;
#pragma unroll
      for (int k0 = 0; k0 < 64; k0 += 16) {
        const bf16x8 ac = frag_rm(sR + C * 32 * LDB + k0, LDB);  // rows c
        const bf16x8 bh = frag_rm(sXh + R * 32 * LDB + k0, LDB), bl = frag_rm(sXl + R * 32 * LDB + k0, LDB);
        if (kside) {
          dTk = mfma(ac, bh, dTk);
          dTk = mfma(ac, bl, dTk);
          kk = mfma(frag_rm(sR + R * 32 * LDB + k0, LDB), ac, kk);  // K K^T, rows r, cols c
        } else {
          dTv = mfma(ac, bh, dTv);
          dTv = mfma(ac, bl, dTv);
        }
      }
    }
    __syncthreads();
  }
  // dT (transposed orientation: rows c, cols r), masked r > c, written back as dT [r][c]
  if (w < 3) {
    f32x16 d;
    const int r = R * 32 + acc_col();
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int c = C * 32 + acc_row(i);
      d[i] = (r > c) ? (dTk[i] * sGam[c] + dTv[i]) * sBeta[c] : 0.f;
    }
    acc_to_lds_t(d, sDh + R * 32 * LDB, sDl + R * 32 * LDB, LDB, C * 32);
  } else {
    acc_to_lds_t(zero16(), sDh, sDl, LDB, 32);  // dT[0..31][32..63] = 0
  }
  __syncthreads();

  // ---- phase 2: M1 = dT T^T (rows r, cols c), masked, stored as M1^T [c][r]
  if (w < 3) {
    f32x16 m = zero16();
#pragma unroll
    for (int k0 = 0; k0 < BT; k0 += 16) {
      const bf16x8 ah = frag_rm(sDh + R * 32 * LDB + k0, LDB), al = frag_rm(sDl + R * 32 * LDB + k0, LDB);
      const bf16x8 bh = frag_rm(sTh + C * 32 * LDB + k0, LDB);
      m = mfma(ah, bh, m);
      m = mfma(ah, frag_rm(sTl + C * 32 * LDB + k0, LDB), m);
      m = mfma(al, bh, m);
    }
    const int c = C * 32 + acc_col();
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (R * 32 + acc_row(i) <= c) m[i] = 0.f;
    acc_to_lds_t(m, sMh + C * 32 * LDB, sMl + C * 32 * LDB, LDB, R * 32);
  } else {
    acc_to_lds_t(zero16(), sMh + 32 * LDB, sMl + 32 * LDB, LDB, 0);  // M1^T[32..63][0..31] = 0
  }
  __syncthreads();
  f32x16 dA = zero16(), dAT = zero16();
  if (w < 3) {
#pragma unroll
    for (int k0 = 0; k0 < BT; k0 += 16) {
      const bf16x8 th = frag_rm(sTth + R * 32 * LDB + k0, LDB), tl = frag_rm(sTtl + R * 32 * LDB + k0, LDB);
      const bf16x8 mh = frag_rm(sMh + C * 32 * LDB + k0, LDB), ml = frag_rm(sMl + C * 32 * LDB + k0, LDB);
      dA = mfma(th, mh, dA);   // rows r, cols c
      dA = mfma(th, ml, dA);
      dA = mfma(tl, mh, dA);
      dAT = mfma(mh, th, dAT);  // rows c, cols r
      dAT = mfma(mh, tl, dAT);
      dAT = mfma(ml, th, dAT);
    }
  }
  __syncthreads();  // scratch (dT, M1^T) is reused below

  // ---- phase 3
  if (w < 3) {
    f32x16 ds;
    const int c = C * 32 + acc_col();
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = R * 32 + acc_row(i);
      const bool keep = r > c;
      const float gam = keep ? __expf(sG[r] - sG[c]) : 0.f;
      const float e = keep ? -dA[i] * gam * kk[i] : 0.f;  // dA = -(T^T M1)
      sE1[r * LDE + c] = e;
      sE2[r * LDE + c] = sBeta[r] * e;
      ds[i] = keep ? -dA[i] * sBeta[r] * gam : 0.f;
    }
    acc_to_lds_t(ds, sATh + C * 32 * LDB, sATl + C * 32 * LDB, LDB, R * 32);  // dAs^T [c][r]
    const int r = R * 32 + acc_col();
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int cc = C * 32 + acc_row(i);
      const bool keep = r > cc;
      ds[i] = keep ? -dAT[i] * sBeta[r] * __expf(sG[r] - sG[cc]) : 0.f;
    }
    acc_to_lds_t(ds, sAh + R * 32 * LDB, sAl + R * 32 * LDB, LDB, C * 32);  // dAs [r][c]
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      sE1[acc_row(i) * LDE + 32 + acc_col()] = 0.f;
      sE2[acc_row(i) * LDE + 32 + acc_col()] = 0.f;
    }
    acc_to_lds_t(zero16(), sATh + 32 * LDB, sATl + 32 * LDB, LDB, 0);
    acc_to_lds_t(zero16(), sAh, sAl, LDB, 32);
  }
  __syncthreads();
  if (tid < 64) {
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < 64; q += 4) {
      const f32x4 x = *(const f32x4*)(sE1 + tid * LDE + q);
      s += x[0] + x[1] + x[2] + x[3];
    }
    sRow[tid] = s;
  } else if (tid < 128) {
    float s = 0.f;
#pragma unroll 8
    for (int i = 0; i < 64; ++i) s += sE2[i * LDE + tid - 64];
    sCol[tid - 64] = s;
  }
  __syncthreads();
  if (tid < BT) {
    sDB[tid] += sRow[tid];
    sDG[tid] += sBeta[tid] * sRow[tid] - sCol[tid];
  }

  // ---- phase 4: dk tiles
  const int tr = (w >> 1) * 32, tc = (w & 1) * 32;
  for (int kt = 0; kt < nkt; ++kt, ++job) {
    pB.store_t(sCt, LDB, L, tid);
    pF.store_t(sFh, sFl, LDB, L, tid);
    pF2.store_rm_f32(sKp, LDE, L, tid);
    __syncthreads();
    if (job + 1 < njobs) issue(job + 1);
    f32x16 acc = zero16(), acc2 = zero16();
#pragma unroll
    for (int k0 = 0; k0 < BT; k0 += 16) {
      const bf16x8 kb = frag_rm(sCt + tc * LDB + k0, LDB);
      acc = mfma(frag_rm(sAh + tr * LDB + k0, LDB), kb, acc);
      acc = mfma(frag_rm(sAl + tr * LDB + k0, LDB), kb, acc);
      acc = mfma(frag_rm(sATh + tr * LDB + k0, LDB), kb, acc);
      acc = mfma(frag_rm(sATl + tr * LDB + k0, LDB), kb, acc);
      const bf16x8 th = frag_rm(sTth + tr * LDB + k0, LDB);
      const bf16x8 fh = frag_rm(sFh + tc * LDB + k0, LDB);
      acc2 = mfma(th, fh, acc2);
      acc2 = mfma(th, frag_rm(sFl + tc * LDB + k0, LDB), acc2);
      acc2 = mfma(frag_rm(sTtl + tr * LDB + k0, LDB), fh, acc2);
    }
    const int c = tc + acc_col(), r0 = tr + acc_row(0);
    float* dk = a.dk32 + (tok0 + r0) * rsk + (long)h * K + kt * 64 + c;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int i4 = tr + acc_row(4 * g);
      const bf16x4 k4 = *(const bf16x4*)(sCt + c * LDB + i4);
      const f32x4 bg = *(const f32x4*)(sBeta + i4), gm = *(const f32x4*)(sGam + i4);
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int kx = 4 * g + ii, r = i4 + ii;
        sE[r * LDE + c] = acc2[kx] * (float)k4[ii];
        if (r < L) dk[acc_drow(kx) * rsk] = sKp[r * LDE + c] + acc[kx] + bg[ii] * gm[ii] * acc2[kx];
      }
    }
    __syncthreads();
    if (tid < 64) {
      float s = 0.f;
#pragma unroll
      for (int q = 0; q < 64; q += 4) {
        const f32x4 x = *(const f32x4*)(sE + tid * LDE + q);
        s += x[0] + x[1] + x[2] + x[3];
      }
      sDB[tid] += sGam[tid] * s;
      sDG[tid] += sBeta[tid] * sGam[tid] * s;
    }
    __syncthreads();
  }
  // ---- phase 5: dv tiles
  for (int vt = 0; vt < nv; ++vt, ++job) {
    pB.store_rm(sCt, LDB, L, tid);
    pF.store_t(sFh, sFl, LDB, L, tid);
    __syncthreads();
    if (job + 1 < njobs) issue(job + 1);
    f32x16 acc = zero16();
#pragma unroll
    for (int k0 = 0; k0 < BT; k0 += 16) {
      const bf16x8 th = frag_rm(sTth + tr * LDB + k0, LDB);
      const bf16x8 fh = frag_rm(sFh + tc * LDB + k0, LDB);
      acc = mfma(th, fh, acc);
      acc = mfma(th, frag_rm(sFl + tc * LDB + k0, LDB), acc);
      acc = mfma(frag_rm(sTtl + tr * LDB + k0, LDB), fh, acc);
    }
    const int c = tc + acc_col(), r0 = tr + acc_row(0);
    bf16* dv = (bf16*)a.dv + (tok0 + r0) * rsv + (long)h * V + vt * 64 + c;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = r0 + acc_drow(i);
      sE[r * LDE + c] = acc[i] * (float)sCt[r * LDB + c];
      if (r < L) gmem(dv)[acc_drow(i) * rsv] = (bf16)(sBeta[r] * acc[i]);
    }
    __syncthreads();
    if (tid < 64) {
      float s = 0.f;
#pragma unroll
      for (int q = 0; q < 64; q += 4) {
        const f32x4 x = *(const f32x4*)(sE + tid * LDE + q);
        s += x[0] + x[1] + x[2] + x[3];
      }
      sDB[tid] += s;
    }
    __syncthreads();
  }
  // ---- dg = reverse cumulative sum of dG within the chunk; dbeta
  if (w == 0) {
    const int ll = lane_id();
    const int r = BT - 1 - ll;  // reverse order
    float x = (r < L) ? sDG[r] : 0.f;
    x = wave_scan_incl(x);
    if (r < L) {
      a.dg[(tok0 + r) * a.H + h] = x;
      a.dbeta[(tok0 + r) * a.H + h] = sDB[r];
    }
  }
}

// ===========================================================================
// gdn_bwd_wy for K, V in {64, 128}: persistent workgroups of 8 waves, one per CU, each taking the
// (chunk, head) units blockIdx.x, blockIdx.x + gridDim.x, ...  Waves 4-7 load the next unit's
// inputs (dw, dU, k, v, T, g, beta, dG partials) into registers while waves 0-3 work on the current
// one, and write them into LDS as soon as the current unit no longer reads that buffer; every
// operand of a unit is read from LDS only (one HBM read of each input).  Per unit, with 32x32 MFMA
// tiles (waves 0-2 take the three lower 32x32 blocks (R, C) of a 64x64 matrix):
//   P1  dT^T blocks (rows c, cols r) over k and v, K K^T in both orientations; dT [r][c] (masked
//       r > c, scaled by beta_c (gamma_c k-part + v-part)) to LDS
//   P2  M1 = dT T^T (masked r > c) to LDS as M1^T;  dA and dA^T = T^T M1 in both orientations
//       (T^T fragments by transposing reads of T)
//   P3  the dbeta / dG terms of A (row sums from dA^T, column sums from dA, both within a lane);
//       dAs + dAs^T (symmetric, zero diagonal) to LDS
//   P4  dk^T tiles: K^T (dAs + dAs^T) + (T^T dw)^T, plus dk_part (read by the compute waves
//       just before P4); dk rows leave as 16-byte pieces; dbeta / dG terms of w
//   P5  dv^T tiles: (T^T dU)^T; dv rows as 8-byte pieces; dbeta terms of u  (the next unit's dw
//       and k are staged meanwhile)
// Barriers per unit: B0 (staged), B1 (dT), B2 (M1^T), B3 (dAs), B4 (dw, k free), B5 (all free).
// The memory waves issue the next unit's loads in two groups (after B0: dw, k; after B2: dU, v, T
// and the per-token values), each ahead of a long compute phase, so issuing them (which stalls
// while the memory system is busy) does not hold a barrier, and each lands well before its staging.
// The compute waves run the key part of P1 (k and dw are staged before B5) ahead of B0, while the
// memory waves stage the value side.  Loops keep several independent accumulators and load the next step's fragments before
// the current step's MFMAs.  Per-row partial sums go to per-wave LDS slots and are added in a fixed
// order (deterministic).
// ===========================================================================
template <int K, int V>
__global__ __launch_bounds__(kWalk8) void gdn_bwd_wy_v3_kernel(const GdnArgs a) {
  constexpr int PT = BT + 8, PK = K + 8, PV = V + 8, NM = 256;
  constexpr int NKB = K / 32, NVB = V / 32;  // 32-column blocks of dk and dv
  constexpr int NJK = NKB / 2, NJV = NVB / 2;  // dk / dv tiles per wave
  // dw and the state part of dk arrive as int16 rows with a scale per 32 columns (dkp_sc / dw_sc)
  // from the K = V = 128 dq/dk/dw kernel, else as fp32
  constexpr bool G16 = K == 128 && V == 128;
  static_assert(NKB % 2 == 0 && NVB % 2 == 0, "two column groups of tiles");
  __shared__ __attribute__((aligned(16))) bf16 sTh[BT * PT], sTl[BT * PT];  // T [a][c]
  __shared__ __attribute__((aligned(16))) bf16 sXh[BT * PT], sXl[BT * PT];  // dT [r][c], then dAs + dAs^T
  __shared__ __attribute__((aligned(16))) bf16 sMh[BT * PT], sMl[BT * PT];  // M1^T [c][r]
  __shared__ __attribute__((aligned(16))) bf16 sWh[BT * PK], sWl[BT * PK];  // dw [t][k]
  __shared__ __attribute__((aligned(16))) bf16 sK[BT * PK];                 // k [t][k]
  __shared__ __attribute__((aligned(16))) bf16 sUh[BT * PV], sUl[BT * PV];  // dU [t][v]
  __shared__ __attribute__((aligned(16))) bf16 sV[BT * PV];                 // v [t][v]
  __shared__ __attribute__((aligned(16))) float sG[BT], sBeta[BT], sGam[BT];
  __shared__ __attribute__((aligned(16))) float sDG0[2 * BT];               // summed dG partials, by unit parity
  __shared__ __attribute__((aligned(16))) float sPB[4 * BT], sPG[4 * BT];  // per compute wave: dbeta, dG terms

  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(wave_id()), l = lane_id();
  const int nunits = a.NTG * a.H;
  const long rsk = (long)a.H * K, rsv = (long)a.H * V;
  const long ntok = a.cu ? (long)a.cu[a.N] : (long)a.N * a.T;
  // first unit at or after u on this workgroup's stride that is not a padding entry of a varlen
  // launch (both roles walk the same sequence)
  auto valid_from = [&](int u) {
    for (; u < nunits; u += gridDim.x) {
      int n, c0, L;
      long bos;
      if (chunk_info(a, u / a.H, n, c0, bos, L)) break;
    }
    return u;
  };

  if (w >= 4) {
    // ---------------- memory waves
    const int lm = tid - NM;
    std::conditional_t<G16, RowsQ16<K, BT, NM>, RowsF32<K, BT, NM>> pw;
    RowsF32<V, BT, NM> pu;
    RowsF32<BT, BT, NM> pt;
    RowsBf16<K, BT, NM> pk;
    RowsBf16<V, BT, NM> pv;
    // per-token values of token l, kept as loaded (used at staging: consuming them earlier would make
    // the wait for them cover the tile loads issued before them)
    float pg = 0.f, pb = 0.f, pd[K / 64];
    int L = 0;
    long tok0 = 0;
    int gc = 0, h = 0;
    auto locate = [&](int u) {
      gc = u / a.H;
      h = u % a.H;
      int n, c0;
      long bos;
      chunk_info(a, gc, n, c0, bos, L);
      tok0 = bos + c0;
    };
    auto load_a = [&]() {
      if constexpr (G16)
        pw.load((const short*)a.dw32 + (tok0 * a.H + h) * K, a.dw_sc + (tok0 * a.H + h) * (K / 32), rsk, rsk / 32, L, lm);
      else
        pw.load(a.dw32 + (tok0 * a.H + h) * K, rsk, L, lm);
      pk.load((const bf16*)a.k + (tok0 * a.H + h) * K, rsk, L, lm);
    };
    auto load_b = [&]() { pu.load(a.dU + (tok0 * a.H + h) * (long)V, rsv, L, lm); };
    auto load_c = [&]() {
      pv.load((const bf16*)a.v + (tok0 * a.H + h) * (long)V, rsv, L, lm);
      pt.load(a.tmat + ((long)gc * a.H + h) * (BT * BT), BT, BT, lm);
      const long tk = (tok0 + min(l, L - 1)) * a.H + h;
      pg = *gmem(a.gcum + tk);
      pb = *gmem(a.beta + tk);
#pragma unroll
      for (int kt = 0; kt < K / 64; ++kt) pd[kt] = *gmem(a.dgp + (long)kt * ntok * a.H + tk);
    };
    auto stage_a = [&]() {
      pw.store_split(sWh, sWl, PK, L, lm);
      pk.store(sK, PK, L, lm);
    };
    // g of token l (the last token's beyond the chunk); beta and the summed dG partials 0 beyond it
    auto stage_b = [&](int par) {
      pu.store_split(sUh, sUl, PV, L, lm);
      pv.store(sV, PV, L, lm);
      pt.store_split(sTh, sTl, PT, BT, lm);
      if (w == 4) {
        float d = 0.f;
#pragma unroll
        for (int kt = 0; kt < K / 64; ++kt) d += pd[kt];
        sG[l] = pg;
        sGam[l] = __expf(pg);
        sBeta[l] = l < L ? pb : 0.f;
        sDG0[par * BT + l] = l < L ? d : 0.f;
      }
    };
    int u = valid_from(blockIdx.x), par = 0;
    if (u < nunits) {
      locate(u);
      load_a();
      load_b();
      load_c();
      stage_a();
      stage_b(0);
    }
    int un = u < nunits ? valid_from(u + gridDim.x) : nunits;
    while (u < nunits) {
      const bool more = un < nunits;
      if (more) locate(un);
      __syncthreads();  // B0
      if (more) load_a();
      __syncthreads();  // B1
      __syncthreads();  // B2
      if (more) {
        load_b();
        load_c();
      }
      __syncthreads();  // B3
      __syncthreads();  // B4
      if (more) stage_a();
      __syncthreads();  // B5
      if (more) stage_b(par ^ 1);
      u = un;
      par ^= 1;
      un = u < nunits ? valid_from(u + gridDim.x) : nunits;
    }
    return;
  }

  // ---------------- compute waves
  const int R = blk_row3(w), C = blk_col3(w);  // lower 32 x 32 block of waves 0..2
  const int tr = w >> 1;                       // 32-row block of this wave's dk / dv tiles
  const int rr = tr * 32 + acc_col();          // the lane's row in dk^T / dv^T tiles
  const int q4 = 4 * (l >> 5);                 // first row of the lane's 4-row groups in a C tile
  int par = 0;
  bool first = true;
  for (int u = valid_from(blockIdx.x); u < nunits; u = valid_from(u + gridDim.x), par ^= 1) {
    const int gc = u / a.H, h = u % a.H;
    int n, c0, L;
    long bos;
    chunk_info(a, gc, n, c0, bos, L);
    const long tok0 = bos + c0;
    // ---- P1, key part: K_c dw_r^T and K K^T both ways.  k and dw of a unit are staged before the
    // previous unit's B5, so this runs ahead of B0 (which waits for the value-side staging); the
    // first unit's operands are all staged before its B0.
    f32x16 kk = zero16(), kkT = zero16(), dTkh = zero16(), dTkl = zero16();
    auto p1_key = [&]() {
      if (w < 3) {
        bf16x8 fa[2][4];
        auto ld = [&](int s, bf16x8* f) {
          f[0] = frag_rm(sK + C * 32 * PK + 16 * s, PK);
          f[1] = frag_rm(sK + R * 32 * PK + 16 * s, PK);
          f[2] = frag_rm(sWh + R * 32 * PK + 16 * s, PK);
          f[3] = frag_rm(sWl + R * 32 * PK + 16 * s, PK);
        };
        ld(0, fa[0]);
#pragma unroll
        for (int s = 0; s < K / 16; ++s) {
          if (s + 1 < K / 16) ld(s + 1, fa[(s + 1) & 1]);
          const bf16x8* f = fa[s & 1];
          dTkh = mfma(f[0], f[2], dTkh);
          kkT = mfma(f[0], f[1], kkT);
          dTkl = mfma(f[0], f[3], dTkl);
          kk = mfma(f[1], f[0], kk);
        }
      }
    };
    if (first) {
      __syncthreads();  // B0: the unit's operands are in LDS
      p1_key();
    } else {
      p1_key();
      __syncthreads();  // B0: the value-side operands are in LDS
    }
    first = false;
    sPB[w * BT + l] = 0.f;
    sPG[w * BT + l] = 0.f;

    // ---- P1, value part: dT^T (rows c, cols r) = K_c dw_r^T gamma_c + V_c dU_r^T
    if (w < 3) {
      f32x16 dTvh = zero16(), dTvl = zero16();
      bf16x8 fa[2][3];
      auto ld = [&](int s, bf16x8* f) {
        f[0] = frag_rm(sV + C * 32 * PV + 16 * s, PV);
        f[1] = frag_rm(sUh + R * 32 * PV + 16 * s, PV);
        f[2] = frag_rm(sUl + R * 32 * PV + 16 * s, PV);
      };
      ld(0, fa[0]);
#pragma unroll
      for (int s = 0; s < V / 16; ++s) {
        if (s + 1 < V / 16) ld(s + 1, fa[(s + 1) & 1]);
        const bf16x8* f = fa[s & 1];
        dTvh = mfma(f[0], f[1], dTvh);
        dTvl = mfma(f[0], f[2], dTvl);
      }
      f32x16 d;
      const int r = R * 32 + acc_col();
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c = C * 32 + 8 * q + q4;
        const f32x4 gm = *(const f32x4*)(sGam + c), bt = *(const f32x4*)(sBeta + c);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const int i = 4 * q + ii;
          d[i] = (r > c + ii) ? ((dTkh[i] + dTkl[i]) * gm[ii] + dTvh[i] + dTvl[i]) * bt[ii] : 0.f;
        }
      }
      acc_to_lds_t(d, sXh + R * 32 * PT, sXl + R * 32 * PT, PT, C * 32);
    } else {
      acc_to_lds_t(zero16(), sXh, sXl, PT, 32);  // dT[0..31][32..63] = 0
    }
    __syncthreads();  // B1

    // ---- P2: M1 = dT T^T (rows r, cols c), masked to r > c, to LDS as M1^T [c][r]
    if (w < 3) {
      f32x16 m1 = zero16(), m2 = zero16();
      bf16x8 fa[2][4];
      auto ld = [&](int s, bf16x8* f) {
        f[0] = frag_rm(sXh + R * 32 * PT + 16 * s, PT);
        f[1] = frag_rm(sXl + R * 32 * PT + 16 * s, PT);
        f[2] = frag_rm(sTh + C * 32 * PT + 16 * s, PT);
        f[3] = frag_rm(sTl + C * 32 * PT + 16 * s, PT);
      };
      ld(0, fa[0]);
#pragma unroll
      for (int s = 0; s < BT / 16; ++s) {
        if (s + 1 < BT / 16) ld(s + 1, fa[(s + 1) & 1]);
        const bf16x8* f = fa[s & 1];
        m1 = mfma(f[0], f[2], m1);
        m2 = mfma(f[0], f[3], m2);
        m1 = mfma(f[1], f[2], m1);
      }
      const int c = C * 32 + acc_col();
#pragma unroll
      for (int i = 0; i < 16; ++i) m1[i] = (R * 32 + acc_row(i) > c) ? m1[i] + m2[i] : 0.f;
      acc_to_lds_t(m1, sMh + C * 32 * PT, sMl + C * 32 * PT, PT, R * 32);
    } else {
      acc_to_lds_t(zero16(), sMh + 32 * PT, sMl + 32 * PT, PT, 0);  // M1^T[32..63][0..31] = 0
    }
    __syncthreads();  // B2

    // ---- P2 (cont.): dA = T^T M1 (rows r, cols c) and dA^T (rows c, cols r); P3
    if (w < 3) {
      f32x16 dA = zero16(), dAT = zero16(), dA2 = zero16(), dAT2 = zero16();
      bf16x8 fa[2][4];
      auto ld = [&](int s, bf16x8* f) {
        f[0] = frag32_tr(sTh + 16 * s * PT + R * 32, PT);
        f[1] = frag32_tr(sTl + 16 * s * PT + R * 32, PT);
        f[2] = frag_rm(sMh + C * 32 * PT + 16 * s, PT);
        f[3] = frag_rm(sMl + C * 32 * PT + 16 * s, PT);
      };
      ld(0, fa[0]);
#pragma unroll
      for (int s = 0; s < BT / 16; ++s) {
        if (s + 1 < BT / 16) ld(s + 1, fa[(s + 1) & 1]);
        const bf16x8* f = fa[s & 1];
        dA = mfma(f[0], f[2], dA);
        dAT = mfma(f[2], f[0], dAT);
        dA2 = mfma(f[0], f[3], dA2);
        dAT2 = mfma(f[2], f[1], dAT2);
        dA = mfma(f[1], f[2], dA);
        dAT = mfma(f[3], f[0], dAT);
      }
      // the true dA is -(T^T M1); e = dA o Gamma o (K K^T), dAs = dA o beta_r Gamma (r > c)
      f32x16 ds1, ds2;
      float srow = 0.f, scol = 0.f;
      {
        const int r = R * 32 + acc_col();
        const float gr_ = sG[r], br_ = sBeta[r];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int c = C * 32 + 8 * q + q4;
          const f32x4 gcv = *(const f32x4*)(sG + c);
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const int i = 4 * q + ii;
            const bool keep = r > c + ii;
            const float x = -(dAT[i] + dAT2[i]);
            const float gam = __expf(keep ? gr_ - gcv[ii] : 0.f);
            srow += keep ? x * gam * kkT[i] : 0.f;
            ds1[i] = keep ? x * br_ * gam : 0.f;
          }
        }
      }
      {
        const int c = C * 32 + acc_col();
        const float gc_ = sG[c];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int r = R * 32 + 8 * q + q4;
          const f32x4 grv = *(const f32x4*)(sG + r), brv = *(const f32x4*)(sBeta + r);
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const int i = 4 * q + ii;
            const bool keep = r + ii > c;
            const float x = -(dA[i] + dA2[i]);
            const float gam = __expf(keep ? grv[ii] - gc_ : 0.f);
            scol += keep ? x * gam * kk[i] * brv[ii] : 0.f;
            ds2[i] = keep ? x * brv[ii] * gam : 0.f;
          }
        }
      }
      srow += __shfl_xor(srow, 32);
      scol += __shfl_xor(scol, 32);
      // dAs at (r, c) from ds1 and at (c, r) from ds2: one symmetric operand; on a diagonal block both
      // land in the same lane and element, so they are added first
      if (R == C) {
#pragma unroll
        for (int i = 0; i < 16; ++i) ds1[i] += ds2[i];
        acc_to_lds_t(ds1, sXh + R * 32 * PT, sXl + R * 32 * PT, PT, C * 32);
      } else {
        acc_to_lds_t(ds1, sXh + R * 32 * PT, sXl + R * 32 * PT, PT, C * 32);
        acc_to_lds_t(ds2, sXh + C * 32 * PT, sXl + C * 32 * PT, PT, R * 32);
      }
      if (l < 32) {
        sPB[w * BT + R * 32 + l] += srow;
        sPG[w * BT + R * 32 + l] += sBeta[R * 32 + l] * srow;
        sPG[w * BT + C * 32 + l] -= scol;
      }
    }
    // dk_part of this wave's dk tiles (rows past the chunk read row L - 1), used at the end of P4;
    // issued before the barrier so that the compiler cannot move them next to their use
    f32x4 dkp[G16 ? 1 : NJK][4];
    s16x4 dkq[G16 ? NJK : 1][4];  // (int16 form: the values and their scale per 32-column block)
    float dks[G16 ? NJK : 1];
    if constexpr (G16) {
      const long row = tok0 + min(rr, L - 1);
#pragma unroll
      for (int j = 0; j < NJK; ++j) {
        dks[j] = *gmem(a.dkp_sc + row * (rsk / 32) + (long)h * (K / 32) + (w & 1) * NJK + j);
#pragma unroll
        for (int g = 0; g < 4; ++g)
          dkq[j][g] = *gmem((const s16x4*)((const short*)a.dkp32 + row * rsk + (long)h * K +
                                           ((w & 1) * NJK + j) * 32 + 8 * g + q4));
      }
    } else {
#pragma unroll
      for (int j = 0; j < NJK; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          dkp[j][g] = *gmem((const f32x4*)(a.dkp32 + (tok0 + min(rr, L - 1)) * rsk + (long)h * K +
                                           ((w & 1) * NJK + j) * 32 + 8 * g + q4));
    }
    __syncthreads();  // B3

    // the unit's dk / dv rows as buffers ending after row L - 1 (stores of later rows are dropped)
    const __amdgpu_buffer_rsrc_t rdk = buf_rsrc(a.dk32 + (tok0 * a.H + h) * K, (int)(((L - 1) * rsk + K) * 4));
    const __amdgpu_buffer_rsrc_t rdv =
        buf_rsrc((const bf16*)a.dv + (tok0 * a.H + h) * (long)V, (int)(((L - 1) * rsv + V) * 2));
    const float br = sBeta[rr], gmr = sGam[rr];
    float s4 = 0.f, s5 = 0.f;
    // ---- P4: dk^T tiles (rows kk, cols r); the dAs and T fragments are shared by the wave's tiles
    {
      f32x16 acc[NJK], acc2[NJK];
#pragma unroll
      for (int j = 0; j < NJK; ++j) acc[j] = acc2[j] = zero16();
      bf16x8 fa[2][4 + 3 * NJK];
      auto ld = [&](int s, bf16x8* f) {
        f[0] = frag_rm(sXh + tr * 32 * PT + 16 * s, PT);
        f[1] = frag_rm(sXl + tr * 32 * PT + 16 * s, PT);
        f[2] = frag32_tr(sTh + 16 * s * PT + tr * 32, PT);
        f[3] = frag32_tr(sTl + 16 * s * PT + tr * 32, PT);
#pragma unroll
        for (int j = 0; j < NJK; ++j) {
          const int tc = (w & 1) * NJK + j;
          f[4 + 3 * j] = frag32_tr(sK + 16 * s * PK + tc * 32, PK);
          f[5 + 3 * j] = frag32_tr(sWh + 16 * s * PK + tc * 32, PK);
          f[6 + 3 * j] = frag32_tr(sWl + 16 * s * PK + tc * 32, PK);
        }
      };
      ld(0, fa[0]);
#pragma unroll
      for (int s = 0; s < BT / 16; ++s) {
        if (s + 1 < BT / 16) ld(s + 1, fa[(s + 1) & 1]);
        const bf16x8* f = fa[s & 1];
#pragma unroll
        for (int j = 0; j < NJK; ++j) {
          acc[j] = mfma(f[4 + 3 * j], f[0], acc[j]);
          acc2[j] = mfma(f[5 + 3 * j], f[2], acc2[j]);
        }
#pragma unroll
        for (int j = 0; j < NJK; ++j) {
          acc[j] = mfma(f[4 + 3 * j], f[1], acc[j]);
          acc2[j] = mfma(f[5 + 3 * j], f[3], acc2[j]);
        }
#pragma unroll
        for (int j = 0; j < NJK; ++j) acc2[j] = mfma(f[6 + 3 * j], f[2], acc2[j]);
      }
#pragma unroll
      for (int j = 0; j < NJK; ++j) {
        const int tc = (w & 1) * NJK + j;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int kc = tc * 32 + 8 * g + q4;
          const bf16x4 k4 = *(const bf16x4*)(sK + rr * PK + kc);
          f32x4 o;
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const int i = 4 * g + ii;
            const float t2 = acc2[j][i];
            const float part = G16 ? dks[j] * (float)dkq[j][g][ii] : dkp[G16 ? 0 : j][g][ii];
            o[ii] = part + acc[j][i] + br * gmr * t2;
            s4 += t2 * (float)k4[ii];
          }
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), rdk, (int)((rr * rsk + kc) * 4), 0, 0);
        }
      }
    }
    __syncthreads();  // B4: dw and k are free (the memory waves stage the next unit's)

    // ---- P5: dv^T tiles (rows v, cols r)
    {
      f32x16 acc[NJV], acc2[NJV];
#pragma unroll
      for (int j = 0; j < NJV; ++j) acc[j] = acc2[j] = zero16();
      bf16x8 fa[2][2 + 2 * NJV];
      auto ld = [&](int s, bf16x8* f) {
        f[0] = frag32_tr(sTh + 16 * s * PT + tr * 32, PT);
        f[1] = frag32_tr(sTl + 16 * s * PT + tr * 32, PT);
#pragma unroll
        for (int j = 0; j < NJV; ++j) {
          const int tc = (w & 1) * NJV + j;
          f[2 + 2 * j] = frag32_tr(sUh + 16 * s * PV + tc * 32, PV);
          f[3 + 2 * j] = frag32_tr(sUl + 16 * s * PV + tc * 32, PV);
        }
      };
      ld(0, fa[0]);
#pragma unroll
      for (int s = 0; s < BT / 16; ++s) {
        if (s + 1 < BT / 16) ld(s + 1, fa[(s + 1) & 1]);
        const bf16x8* f = fa[s & 1];
#pragma unroll
        for (int j = 0; j < NJV; ++j) {
          acc[j] = mfma(f[2 + 2 * j], f[0], acc[j]);
          acc2[j] = mfma(f[2 + 2 * j], f[1], acc2[j]);
        }
#pragma unroll
        for (int j = 0; j < NJV; ++j) acc[j] = mfma(f[3 + 2 * j], f[0], acc[j]);
      }
#pragma unroll
      for (int j = 0; j < NJV; ++j) {
        const int tc = (w & 1) * NJV + j;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int vc = tc * 32 + 8 * g + q4;
          const bf16x4 v4 = *(const bf16x4*)(sV + rr * PV + vc);
          bf16x4 o;
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const float x = acc[j][4 * g + ii] + acc2[j][4 * g + ii];
            o[ii] = (bf16)(br * x);
            s5 += x * (float)v4[ii];
          }
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, o), rdv, (int)((rr * rsv + vc) * 2), 0, 0);
        }
      }
    }
    s4 += __shfl_xor(s4, 32);
    s5 += __shfl_xor(s5, 32);
    if (l < 32) {
      sPB[w * BT + rr] += gmr * s4 + s5;
      sPG[w * BT + rr] += br * gmr * s4;
    }
    __syncthreads();  // B5: every LDS read of the unit done; the memory waves stage the rest

    // ---- dbeta, and dg = reverse cumulative sum of dG within the chunk
    if (w == 0) {
      const int r = BT - 1 - l;  // reverse order
      float db = 0.f, x = sDG0[par * BT + r];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        db += sPB[q * BT + r];
        x += sPG[q * BT + r];
      }
      if (r >= L) x = 0.f;
      x = wave_scan_incl(x);
      if (r < L) {
        a.dg[(tok0 + r) * a.H + h] = x;
        a.dbeta[(tok0 + r) * a.H + h] = db;
      }
    }
  }
}

// ===========================================================================
// gdn_bwd_dqkw for K = 128, V in {64, 128} and fp32 q_clean (launched for V = 64; V = 128 takes
// the three-slot form below): a persistent kernel, one 8-wave workgroup per CU over the (chunk,
// head) units, same results as gdn_bwd_dqkw_v3_kernel.  The
// operands stream through two 64 KiB LDS slots by direct-to-LDS loads (global_load_lds_dwordx4:
// no registers held, no staging pass): a unit is V/32 value pieces (h and dS' rows [32 v][128 k]
// as hi/lo pairs, U, dU and dO columns [64 t][32 v]) and one post piece (q_clean, k, P^T).  While
// one slot is being computed on, the next piece loads into the other, and the next unit's first
// two pieces load during this unit's post stage.  Each piece is 8 load instructions per wave, so
// "the piece before the newest has landed" is s_waitcnt vmcnt(8) (stores issued in between only
// make that wait longer).  Rows are stored with an XOR swizzle of their 16-byte pieces so that
// the MFMA operand reads (row pieces and ds_read_b64_tr_b16 column reads) are free of bank
// conflicts; rows past the chunk are loaded from its last row and masked in the products.
// Waves: w & 1 = 32-row half of the chunk (tr), w >> 1 = 32-column quarter of K (kc); waves 0, 1
// and 3 also hold the 32 x 32 tiles (0,0), (32,0), (32,32) of dP = dO U^T.  The decay gradient
// is written whole into partial 0 (partial 1 = 0).
// ===========================================================================
namespace dq4 {
constexpr int SLOT = 65536;
// value piece regions (bytes): h, h_lo, dS', dS'_lo [32 v][128 k] bf16; U, dU [64 t][32 v] fp32;
// dO [64 t][32 v] bf16
constexpr int RH = 0, RHL = 8192, RDH = 16384, RDHL = 24576, RU = 32768, RDU = 40960, RDO = 49152;
// post piece regions: q_clean [64 t][128 k] fp32, k [64 t][128 k] bf16, P^T [64 s][64 t] fp32
constexpr int RQ = 0, RK = 32768, RP = 49152;
constexpr int LDP = 80;  // dPs rows (bf16): 160 bytes, conflict-free transposing reads

// Direct-to-LDS loads: wave-uniform global base + 32-bit lane byte offset; lane i's 16 (4) bytes
// land at LDS s + 16 i (4 i), s wave-uniform.  Written as inline assembly so that the compiler does
// not track them: with the builtin it drains all loads (vmcnt(0)) before LDS reads it cannot tell
// apart, which serialises the two slots.  Their completion is waited for by wait_vm alone.  The
// instruction reads M0 one wait state after it is written (the s_nop).
typedef __attribute__((address_space(3))) char lds_char;
__device__ __forceinline__ void dma16(const void* base, unsigned off, char* s) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)(lds_char*)s);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(m0), "v"(off), "s"(base) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* base, unsigned off, char* s) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)(lds_char*)s);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2" ::"s"(m0), "v"(off), "s"(base) : "memory", "m0");
}
// this lane's index through an opaque copy: addresses derived from it are recomputed where they
// are used instead of being merged across the unrolled pieces (which keeps them live throughout)
__device__ __forceinline__ int fresh_lane() {
  int l = threadIdx.x & 63;
  asm volatile("" : "+v"(l));
  return l;
}
// s_waitcnt vmcnt(N) lgkmcnt(0)
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70);
}
// workgroup barrier after this wave's LDS operations completed; a compiler fence on both sides
// (no global wait: the direct-to-LDS loads are waited for by wait_vm)
__device__ __forceinline__ void bar() {
  __builtin_amdgcn_s_waitcnt(0xC07F);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
// Scalar loads of read-only launch tables (varlen offsets): a vector load here would make the
// compiler drain every outstanding load, direct-to-LDS ones included, before its use.
__device__ __forceinline__ int sld_i32(const int* p) {
  int v;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p));
  return v;
}
__device__ __forceinline__ long sld_i64(const int64_t* p) {
  long v;
  asm volatile("s_load_dwordx2 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p));
  return v;
}
// byte offsets of swizzled elements
__device__ __forceinline__ int off_h(int r, int k) {  // bf16 rows of 256 bytes, piece ^= 2 (r & 3)
  return r * 256 + ((((k >> 3) ^ (2 * (r & 3))) << 4) | ((k & 7) << 1));
}
__device__ __forceinline__ int off_u(int r, int v) {  // fp32 rows of 128 bytes, piece ^= r & 7
  return r * 128 + ((((v >> 2) ^ (r & 7)) << 4) | ((v & 3) << 2));
}
__device__ __forceinline__ int off_o(int r, int v) {  // bf16 rows of 64 bytes, piece ^= (r >> 1) & 3
  return r * 64 + ((((v >> 3) ^ ((r >> 1) & 3)) << 4) | ((v & 7) << 1));
}
__device__ __forceinline__ int off_p(int s, int t) {  // fp32 rows of 256 bytes, piece ^= s & 15
  return s * 256 + ((((t >> 2) ^ (s & 15)) << 4) | ((t & 3) << 2));
}
// B operand (contraction down the rows) from a swizzled [rows][128] bf16 region: columns c0 .. +31,
// contraction rows r0 .. +15 (r0 a multiple of 16): two transposing reads (frag32_tr's lane map)
__device__ __forceinline__ bf16x8 frag_tr_h(const char* R, int r0, int c0, int l) {
  const int j = l & 15;
  const int r = r0 + 8 * (l >> 5) + (j >> 2), c = c0 + 16 * ((l >> 4) & 1) + 4 * (j & 3);
  typedef __attribute__((address_space(3))) bf16x4_t lds_b4;
  const char* q = R + off_h(r, c);
  const bf16x4_t x = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_b4*)q);
  const bf16x4_t y = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_b4*)(q + 4 * 256));
  return bf16x8{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
}
// The same B operand from a block-floating-point snapshot region (int16 rows with power-of-two scales;
// sc: the region's 32 row scales, fp32): each element times its row's scale, split into hi/lo bf16
__device__ __forceinline__ void frag_tr_h16(const char* R, const char* sc, int r0, int c0, int l, bf16x8& hi,
                                            bf16x8& lo) {
  const i16x8 x = __builtin_bit_cast(i16x8, frag_tr_h(R, r0, c0, l));
  const int v = r0 + 8 * (l >> 5);
  const f32x4 s0 = *(const f32x4*)(sc + 4 * v), s1 = *(const f32x4*)(sc + 4 * v + 16);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    bf16 h, o;
    split2((float)x[i] * (i < 4 ? s0[i] : s1[i - 4]), h, o);
    hi[i] = h;
    lo[i] = o;
  }
}
// A/B operand rows r0 + l % 32, contraction v0 + 8 (l / 32) .. +7 of a swizzled fp32 [64][32] region,
// split into hi/lo
__device__ __forceinline__ void frag_u(const char* R, int r0, int v0, bf16x8& hi, bf16x8& lo, int l) {
  const int r = r0 + (l & 31), c = (v0 >> 2) + 2 * (l >> 5);
  const f32x4 x = *(const f32x4*)(R + r * 128 + ((c ^ (r & 7)) << 4));
  const f32x4 y = *(const f32x4*)(R + r * 128 + (((c + 1) ^ (r & 7)) << 4));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bf16 h, o;
    split2(x[i], h, o);
    hi[i] = h;
    lo[i] = o;
    split2(y[i], h, o);
    hi[4 + i] = h;
    lo[4 + i] = o;
  }
}
// A operand rows r0 + l % 32, contraction v0 + 8 (l / 32) .. +7 of the swizzled dO region
__device__ __forceinline__ bf16x8 frag_o(const char* R, int r0, int v0, int l) {
  const int r = r0 + (l & 31), c = (v0 >> 3) + (l >> 5);
  return *(const bf16x8*)(R + r * 64 + ((c ^ ((r >> 1) & 3)) << 4));
}
// frag_rm / frag32_tr / acc_row with the lane index passed in
__device__ __forceinline__ bf16x8 frag_rm_l(const bf16* p, int ld, int l) {
  return *(const bf16x8*)(p + (l & 31) * ld + ((l >> 5) << 3));
}
__device__ __forceinline__ bf16x8 frag32_tr_l(const bf16* p, int ld, int l) {
  const int j = l & 15;
  const bf16* q = p + (8 * (l >> 5) + (j >> 2)) * ld + 16 * ((l >> 4) & 1) + 4 * (j & 3);
  typedef __attribute__((address_space(3))) bf16x4_t lds_b4;
  const bf16x4_t x = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_b4*)q);
  const bf16x4_t y = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_b4*)(q + 4 * ld));
  return bf16x8{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
}
__device__ __forceinline__ int arow(int i, int l) { return ((i >> 2) << 3) + ((l >> 5) << 2) + (i & 3); }
// Value held by lane l ^ M, moved by DPP (M < 16) or v_permlane16/32_swap, not through the LDS pipe
// (ds_bpermute waits behind the direct-to-LDS traffic).
template <int C>
__device__ __forceinline__ float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), C, 0xf, 0xf, false));
}
template <int M>
__device__ __forceinline__ float xlane(float x, int l) {
  if constexpr (M == 1) {
    return dpp_mov<0xB1>(x);  // quad_perm [1, 0, 3, 2]
  } else if constexpr (M == 2) {
    return dpp_mov<0x4E>(x);  // quad_perm [2, 3, 0, 1]
  } else if constexpr (M == 4) {
    const float up = dpp_mov<0x104>(x), dn = dpp_mov<0x114>(x);  // row_shl:4 (lane + 4), row_shr:4 (lane - 4)
    return (l & 4) ? dn : up;
  } else if constexpr (M == 8) {
    return dpp_mov<0x128>(x);  // row_ror:8
  } else if constexpr (M == 16) {
    // odd 16-lane rows of the first operand swap with even rows of the second
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, x), __builtin_bit_cast(unsigned, x), false, false);
    return __builtin_bit_cast(float, (l & 16) ? r[0] : r[1]);
  } else {
    static_assert(M == 32, "lane distance");
    // rows 2, 3 of the first operand swap with rows 0, 1 of the second
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x), __builtin_bit_cast(unsigned, x), false, false);
    return __builtin_bit_cast(float, (l & 32) ? r[0] : r[1]);
  }
}
__device__ __forceinline__ float wave_sum(float x, int l) {
  x += xlane<1>(x, l);
  x += xlane<2>(x, l);
  x += xlane<4>(x, l);
  x += xlane<8>(x, l);
  x += xlane<16>(x, l);
  return x + xlane<32>(x, l);
}
// Row sums of a 32 x 32 C tile: reduce-scatter over the 32 lanes of each half-wave.  Returns the
// sum of row acc_row((l >> 1) & 15) (lanes l and l ^ 1 hold the same value).
__device__ __forceinline__ float rowsum32(const f32x16& ev, int l) {
  // the elements as opaque scalars: "c ? v[i] : v[j]" on the vector is otherwise turned into an
  // index chosen at run time, i.e. a 16-way select per element
  float e[16], a8[8], a4[4], a2[2];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    e[i] = ev[i];
    asm volatile("" : "+v"(e[i]));
  }
  const bool b4 = (l >> 4) & 1, b3 = (l >> 3) & 1, b2 = (l >> 2) & 1, b1 = (l >> 1) & 1;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float send = b4 ? e[i] : e[i + 8], keep = b4 ? e[i + 8] : e[i];
    a8[i] = keep + xlane<16>(send, l);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float send = b3 ? a8[i] : a8[i + 4], keep = b3 ? a8[i + 4] : a8[i];
    a4[i] = keep + xlane<8>(send, l);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float send = b2 ? a4[i] : a4[i + 2], keep = b2 ? a4[i + 2] : a4[i];
    a2[i] = keep + xlane<4>(send, l);
  }
  const float send = b1 ? a2[0] : a2[1], keep = b1 ? a2[1] : a2[0];
  const float a1 = keep + xlane<2>(send, l);
  return a1 + xlane<1>(a1, l);
}
// Largest |x| of each of the lane's 16 rows of a 32 x 32 C tile, over the row's 32 columns (the 32
// lanes of the half-wave); every lane ends with the maxima of its own rows.  Integer maxima of the
// magnitudes' bit patterns (as group_umax): after the two quad steps every
// lane of a quad holds the quad's maximum, so rotating the row by 4 and then by 8 brings in the other
// three quads'.
__device__ __forceinline__ f32x16 rowmax32_all(const f32x16& v, int l) {
  f32x16 m;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    unsigned x = __float_as_uint(v[i]) & 0x7fffffffu;
    x = umax_dpp<0xB1>(x);   // quad_perm [1, 0, 3, 2]
    x = umax_dpp<0x4E>(x);   // quad_perm [2, 3, 0, 1]
    x = umax_dpp<0x124>(x);  // row_ror:4
    x = umax_dpp<0x128>(x);  // row_ror:8
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    m[i] = __uint_as_float(max((unsigned)r[0], (unsigned)r[1]));
  }
  return m;
}
// Exponent e of the power-of-two scale of an int16 row piece with largest magnitude mx: mx / 2^e in
// [2^14, 2^15) (floor(log2 mx) from the exponent field; 0 and subnormal maxima land on the lower clamp).
__device__ __forceinline__ int q16_exp(float mx) {
  return min(max((int)((__float_as_uint(mx) >> 23) & 0xff) - 127 - 14, -126), 113);
}
__device__ __forceinline__ unsigned short q16(float x, int e) {
  return (unsigned short)(short)__builtin_amdgcn_fmed3f(rintf(ldexpf(x, -e)), -32767.f, 32767.f);
}
}  // namespace dq4

template <int V>
__global__ __launch_bounds__(kWalk8) void gdn_bwd_dqkw_v4_kernel(const GdnArgs a) {
  using namespace dq4;
  constexpr int K = 128, NP = V / 32;
  static_assert(NP % 2 == 0, "an even number of value pieces: each unit's post piece lands in its first slot");
  __shared__ __attribute__((aligned(1024))) char sA[SLOT];
  __shared__ __attribute__((aligned(1024))) char sB[SLOT];
  __shared__ __attribute__((aligned(16))) bf16 sPh[BT * LDP], sPl[BT * LDP];  // dPs [t][s] hi/lo
  __shared__ __attribute__((aligned(16))) float sGr[8][BT];  // g of the unit's tokens (one copy per wave)
  __shared__ __attribute__((aligned(16))) float sRP[3][32], sCP[3][32];      // dP o P row / column sums per dP tile
  __shared__ __attribute__((aligned(16))) float sRQ[4][BT], sRK[4][BT];      // per K quarter: dQ o q_clean, dK o k
  __shared__ __attribute__((aligned(16))) float sHD[8];

  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(wave_id()), l = lane_id();
  const int tr = 32 * (w & 1), kc = 32 * (w >> 1);
  const int dpi = w == 0 ? 0 : w == 1 ? 1 : w == 3 ? 2 : -1;  // dP tile of this wave
  const int tp = dpi == 0 ? 0 : 32, sp = dpi == 2 ? 32 : 0;
  const int nunits = a.NTG * a.H;
  const long rsk = (long)a.H * K, rsv = (long)a.H * V;
  const long ntok = a.cu ? (long)a.cu[a.N] : (long)a.N * a.T;

  struct Unit {
    int u, gc, h, L;
    long tok0;
  };
  // chunk_info with wave-uniform values and scalar loads
  auto chunk_s = [&](int gc, int& L, long& tok0) {
    if (a.cu) {
      const int n = sld_i32(a.chunk_idx + 2 * gc);
      if (n < 0) return false;
      const int c = sld_i32(a.chunk_idx + 2 * gc + 1);
      const long b0 = sld_i64(a.cu + n), b1 = sld_i64(a.cu + n + 1);
      tok0 = b0 + (long)c * BT;
      L = min(BT, (int)(b1 - b0) - c * BT);
    } else {
      const int n = gc / a.NT, c = gc - n * a.NT;
      tok0 = (long)n * a.T + (long)c * BT;
      L = min(BT, a.T - c * BT);
    }
    return true;
  };
  auto valid_from = [&](int u) {
    for (; u < nunits; u += gridDim.x) {
      int L;
      long t0;
      if (chunk_s(__builtin_amdgcn_readfirstlane(u / a.H), L, t0)) break;
    }
    return u;
  };
  auto locate = [&](int u) {
    Unit x{u, 0, 0, 1, 0};
    if (u < nunits) {
      x.gc = __builtin_amdgcn_readfirstlane(u / a.H);
      x.h = u - x.gc * a.H;
      chunk_s(x.gc, x.L, x.tok0);
    }
    return x;
  };

  // ---- direct-to-LDS loads of one piece: 8 instructions per wave (9 for the post piece)
  auto issue_v = [&](char* S, const Unit& x, int vb) {
    const int v0 = 32 * vb, l = fresh_lane();
    {
      const long ub = (((long)x.gc * a.H + x.h) * V + v0) * K;
      const int r = 4 * w + (l >> 4), p = l & 15;
      const unsigned off = (unsigned)((r * K + 8 * (p ^ (2 * (r & 3)))) * 2);
      dma16((const bf16*)a.hT + ub, off, S + RH + 1024 * w);
      dma16((const bf16*)a.hTl + ub, off, S + RHL + 1024 * w);
      dma16((const bf16*)a.dhT + ub, off, S + RDH + 1024 * w);
      dma16((const bf16*)a.dhTl + ub, off, S + RDHL + 1024 * w);
    }
    const long ub = x.tok0 * rsv + (long)x.h * V + v0;
    {
      const int r = 8 * w + (l >> 3), p = l & 7;
      const unsigned off = (unsigned)((min(r, x.L - 1) * (int)rsv + 4 * (p ^ (r & 7))) * 4);
      dma16(a.U + ub, off, S + RU + 1024 * w);
      dma16(a.dU + ub, off, S + RDU + 1024 * w);
    }
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int j = 2 * w + jj, r = 4 * j + (l >> 4), d = l & 15;
      const unsigned off = (unsigned)((min(r, x.L - 1) * (int)rsv + 8 * ((d >> 2) ^ ((r >> 1) & 3)) + 2 * (d & 3)) * 2);
      dma4((const bf16*)a.dout + ub, off, S + RDO + 256 * j);
    }
  };
  auto issue_p = [&](char* S, const Unit& x) {
    const int l = fresh_lane();
    const long ub = x.tok0 * rsk + (long)x.h * K;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int j = 4 * w + jj, r = 2 * j + (l >> 5);
      const unsigned off = (unsigned)((min(r, x.L - 1) * (int)rsk + 4 * (l & 31)) * 4);
      dma16(a.qc32 + ub, off, S + RQ + 1024 * j);
    }
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int j = 2 * w + jj, r = 4 * j + (l >> 4), p = l & 15;
      const unsigned off = (unsigned)((min(r, x.L - 1) * (int)rsk + 8 * (p ^ (2 * (r & 3)))) * 2);
      dma16((const bf16*)a.k + ub, off, S + RK + 1024 * j);
    }
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int j = 2 * w + jj, s = 4 * j + (l >> 4), p = l & 15;
      const unsigned off = (unsigned)((s * BT + 4 * (p ^ (s & 15))) * 4);
      dma16(a.PT + ((long)x.gc * a.H + x.h) * (BT * BT), off, S + RP + 1024 * j);
    }
    // g of the unit's tokens (the last token's past the chunk), a copy per wave
    dma4(a.gcum + x.tok0 * a.H + x.h, (unsigned)(min(l, x.L - 1) * a.H * 4), (char*)&sGr[w][0]);
  };

  f32x16 dQi, dKs, dW, dP;
  float hds;

  // ---- one value piece: <h, dS'>, dQi += dO h^T, dKs += U dS'^T, dW += dU h^T, dP += dO U^T
  auto compute_v = [&](const char* S) {
    const int l = fresh_lane();
    {
      const int o = 16 * (64 * w + l);
      const bf16x8 x1 = *(const bf16x8*)(S + RH + o), x2 = *(const bf16x8*)(S + RHL + o);
      const bf16x8 y1 = *(const bf16x8*)(S + RDH + o), y2 = *(const bf16x8*)(S + RDHL + o);
#pragma unroll
      for (int i = 0; i < 8; ++i) hds += ((float)x1[i] + (float)x2[i]) * ((float)y1[i] + (float)y2[i]);
    }
#pragma unroll
    for (int v0 = 0; v0 < 32; v0 += 16) {
      const bf16x8 oa = frag_o(S + RDO, tr, v0, l);
      const bf16x8 hb = frag_tr_h(S + RH, v0, kc, l), hbl = frag_tr_h(S + RHL, v0, kc, l);
      const bf16x8 db = frag_tr_h(S + RDH, v0, kc, l), dbl = frag_tr_h(S + RDHL, v0, kc, l);
      bf16x8 uh, ul, dh, dl;
      frag_u(S + RU, tr, v0, uh, ul, l);
      frag_u(S + RDU, tr, v0, dh, dl, l);
      dQi = mfma(oa, hb, dQi);
      dQi = mfma(oa, hbl, dQi);
      dKs = mfma(uh, db, dKs);
      dKs = mfma(ul, db, dKs);
      dKs = mfma(uh, dbl, dKs);
      dW = mfma(dh, hb, dW);
      dW = mfma(dl, hb, dW);
      dW = mfma(dh, hbl, dW);
      if (dpi == 0 || dpi == 2) {
        dP = mfma(oa, uh, dP);
        dP = mfma(oa, ul, dP);
      } else if (dpi == 1) {
        bf16x8 sh, sl;
        frag_u(S + RU, 0, v0, sh, sl, l);
        dP = mfma(oa, sh, dP);
        dP = mfma(oa, sl, dP);
      }
    }
  };

  // ---- post stage on the post piece in S
  auto post = [&](const char* S, const Unit& x) {
    const int L = x.L, l = fresh_lane();
    // dP (waves 0, 1, 3): causal and chunk mask, dPs = scale dP Gamma as hi/lo [t][s], dP o P sums
    if (dpi >= 0) {
      const int c = sp + (l & 31);
      const float gcol = sGr[0][c];
      f32x16 e;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r4 = tp + arow(4 * q, l);
        const f32x4 pv = *(const f32x4*)(S + RP + off_p(c, r4));  // P[r][c] = P^T[c][r]
        const f32x4 gr = *(const f32x4*)&sGr[0][r4];
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const int i = 4 * q + ii, r = r4 + ii;
          const bool keep = r >= c && r < L;
          const float d = keep ? dP[i] : 0.f;
          const float ev = __expf(gr[ii] - gcol);  // (overflow only where masked)
          const float ps = keep ? d * a.scale * ev : 0.f;
          bf16 hi, lo;
          split2(ps, hi, lo);
          sPh[r * LDP + c] = hi;
          sPl[r * LDP + c] = lo;
          e[i] = d * pv[ii];
        }
      }
      float cs = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) cs += e[i];
      cs += xlane<32>(cs, l);
      if (l < 32) sCP[dpi][l] = cs;
      const float rs = rowsum32(e, l);
      if ((l & 1) == 0) sRP[dpi][arow((l >> 1) & 15, l)] = rs;
    }
    // scale the state parts; dG terms sum_k dQ q_clean and sum_k dK k over this wave's columns
    {
      const int c = kc + (l & 31);
      const float gl = sGr[0][L - 1];
      f32x16 e, f, gv;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 g4 = *(const f32x4*)&sGr[0][tr + arow(4 * q, l)];
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) gv[4 * q + ii] = g4[ii];
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = tr + arow(i, l);
        const float g = gv[i];
        dQi[i] *= a.scale * __expf(g);
        e[i] = dQi[i] * *(const float*)(S + RQ + r * 512 + 4 * c);
        dKs[i] *= __expf(gl - g);
        f[i] = dKs[i] * (float)*(const bf16*)(S + RK + off_h(r, c));
      }
      const float re = rowsum32(e, l), rf = rowsum32(f, l);
      if ((l & 1) == 0) {
        const int r = tr + arow((l >> 1) & 15, l);
        sRQ[w >> 1][r] = re;
        sRK[w >> 1][r] = rf;
      }
    }
    {
      const float s = wave_sum(hds, l);
      if (l == 0) sHD[w] = s;
    }
    bar();
    // dq = scale gamma dQi + dPs k (s <= t: the t < 32 half needs s < 32 only)
    {
#pragma unroll
      for (int s0 = 0; s0 < BT; s0 += 16) {
        if (tr == 0 && s0 >= 32) break;
        const bf16x8 kb = frag_tr_h(S + RK, s0, kc, l);
        dQi = mfma(frag_rm_l(sPh + tr * LDP + s0, LDP, l), kb, dQi);
        dQi = mfma(frag_rm_l(sPl + tr * LDP + s0, LDP, l), kb, dQi);
      }
      const auto rs = buf_rsrc(a.dq32 + x.tok0 * rsk + (long)x.h * K, (int)(((L - 1) * rsk + K) * 4));
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = tr + arow(i, l);
        const float x = dQi[i];  // (bit_cast of a vector element reference reads element 0)
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, x), rs, (int)((r * rsk + kc + (l & 31)) * 4), 0, 0);
      }
    }
    // dk = fac dKs + dPs^T q_clean (i >= j: the j >= 32 half needs i >= 32 only); dw = -dW
    {
      const int c = kc + (l & 31);
#pragma unroll
      for (int i0 = 0; i0 < BT; i0 += 16) {
        if (tr == 32 && i0 < 32) continue;
        const bf16x8 ah = frag32_tr_l(sPh + i0 * LDP + tr, LDP, l), al = frag32_tr_l(sPl + i0 * LDP + tr, LDP, l);
        bf16x8 bh, bl;
        const int ib = i0 + 8 * (l >> 5);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          bf16 hh, oo;
          split2(*(const float*)(S + RQ + (ib + e) * 512 + 4 * c), hh, oo);
          bh[e] = hh;
          bl[e] = oo;
        }
        dKs = mfma(ah, bh, dKs);
        dKs = mfma(ah, bl, dKs);
        dKs = mfma(al, bh, dKs);
      }
      const int bytes = (int)(((L - 1) * rsk + K) * 4);
      const auto rk = buf_rsrc(a.dkp32 + x.tok0 * rsk + (long)x.h * K, bytes);
      const auto rw = buf_rsrc(a.dw32 + x.tok0 * rsk + (long)x.h * K, bytes);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = tr + arow(i, l), off = (int)((r * rsk + c) * 4);
        const float xk = dKs[i], xw = -dW[i];
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, xk), rk, off, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, xw), rw, off, 0, 0);
      }
    }
    bar();
    // decay gradient of token t: (dP o P) row t - column t + dQ o q_clean - dK o k; the last token
    // also takes every dK o k term and e^{G_L} <h, dS'>
    if (w == 0) {
      const int t = l;
      const float term = t < L ? sRK[0][t] + sRK[1][t] + sRK[2][t] + sRK[3][t] : 0.f;
      const float tot = wave_sum(term, l);
      if (t < L) {
        float d = t < 32 ? sRP[0][t] - sCP[0][t] - sCP[1][t]
                         : sRP[1][t - 32] + sRP[2][t - 32] - sCP[2][t - 32];
        d += sRQ[0][t] + sRQ[1][t] + sRQ[2][t] + sRQ[3][t] - term;
        if (t == L - 1) {
          float hsum = 0.f;
#pragma unroll
          for (int ww = 0; ww < 8; ++ww) hsum += sHD[ww];
          d += tot + __expf(sGr[0][L - 1]) * hsum;
        }
        const long gi = (x.tok0 + t) * a.H + x.h;
        a.dgp[gi] = d;
        a.dgp[ntok * a.H + gi] = 0.f;
      }
    }
  };

  // ---- one unit: value pieces alternate X, Y, X, ...; the post piece lands in X
  auto unit = [&](char* X, char* Y, const Unit& cur, const Unit& nxt) {
    const bool more = nxt.u < nunits;
    dQi = zero16();
    dKs = zero16();
    dW = zero16();
    dP = zero16();
    hds = 0.f;
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      char* S = (j & 1) ? Y : X;
      if (j == NP - 1) wait_vm<9>();  // the post piece is the newer one in flight
      else wait_vm<8>();
      bar();
      compute_v(S);
      bar();
      if (j + 2 < NP) issue_v(S, cur, j + 2);
      else if (j + 2 == NP) issue_p(S, cur);
      else if (more) issue_v(S, nxt, 0);
    }
    if (more) wait_vm<8>();
    else wait_vm<0>();
    bar();
    post(X, cur);
    bar();
    if (more) issue_v(X, nxt, 1);
  };

  Unit cur = locate(valid_from(blockIdx.x));
  if (cur.u >= nunits) return;
  Unit nxt = locate(valid_from(cur.u + gridDim.x));
  issue_v(sA, cur, 0);
  issue_v(sB, cur, 1);
  while (true) {
    unit(sA, sB, cur, nxt);
    if (nxt.u >= nunits) break;
    cur = nxt;
    nxt = locate(valid_from(cur.u + gridDim.x));
    unit(sB, sA, cur, nxt);
    if (nxt.u >= nunits) break;
    cur = nxt;
    nxt = locate(valid_from(cur.u + gridDim.x));
  }
}

// ===========================================================================
// gdn_bwd_dqkw for K = V = 128 (q_clean fp32 or bf16), three-slot form of gdn_bwd_dqkw_v4_kernel: a
// unit is six pieces in three 52 KiB LDS slots -- value pieces V0 .. V3 (slots 0 1 2 0), then
// q_clean (slot 1) and k with P^T (slot 2; dPs is formed in that slot's tail).  A piece is loaded
// one to two phases ahead, during the compute of an earlier piece (the next unit's V0 during the
// post stage, its V1 as soon as the post stage's products are done), and the load instructions
// are issued between MFMAs (waves 0-3 after the first 16-value step, waves 4-7 after the second),
// so that the two waves of a SIMD stall on issue at different times.  One barrier per piece.
// Loads per wave: value piece 8, q_clean piece 4 fp32 / 2 bf16 (one more on wave 0, which also
// loads g), k/P^T piece 4; the wait before a piece is vmcnt(loads issued after it).  A bf16
// q_clean is stored swizzled like k and read with transposing reads; its lo part is zero.
// The state and state-gradient snapshots arrive as int16 rows with a power-of-two scale per row (the
// walks write that form for K = V = 128: half the bytes of hi/lo pairs); a value piece holds the
// two int16 regions and, in place of their lo parts, each wave's copy of the 32 row scales, so it is
// still 8 load instructions per wave.  The B operands are rebuilt as hi/lo pairs of scale x value.
// ===========================================================================
namespace dq5 {
constexpr int SLOT = 53248;
constexpr int RK = 0, RP = 16384;     // k [64 t][128 k] bf16, P^T [64 s][64 t] fp32
constexpr int RPH = 32768, RPL = RPH + dq4::LDP * BT * 2;  // dPs hi / lo [t][s] in the k/P^T slot
}  // namespace dq5

template <bool Q32>
__global__ __launch_bounds__(kWalk8) void gdn_bwd_dqkw_v5_kernel(const GdnArgs a) {
  using namespace dq4;
  using dq5::SLOT;
  constexpr int K = 128, V = 128;
  __shared__ __attribute__((aligned(1024))) char s0[SLOT];
  __shared__ __attribute__((aligned(1024))) char s1[SLOT];
  __shared__ __attribute__((aligned(1024))) char s2[SLOT];
  __shared__ __attribute__((aligned(16))) float sRP[3][32], sCP[3][32];  // dP o P row / column sums per dP tile
  __shared__ __attribute__((aligned(16))) float sRQ[4][BT], sRK[4][BT];  // per K quarter: dQ o q_clean, dK o k
  __shared__ __attribute__((aligned(16))) float sHD[8];
  __shared__ __attribute__((aligned(16))) float sG[BT];                  // g of the unit's tokens

  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(wave_id());
  const int tr = 32 * (w & 1), kc = 32 * (w >> 1);
  const int dpi = w == 0 ? 0 : w == 1 ? 1 : w == 3 ? 2 : -1;  // dP tile of this wave
  const int tp = dpi == 0 ? 0 : 32, sp = dpi == 2 ? 32 : 0;
  const bool early = w < 4;  // issues its loads after the first 16-value step
  const int nunits = a.NTG * a.H;
  const long rsk = (long)a.H * K, rsv = (long)a.H * V;
  const long ntok = a.cu ? (long)a.cu[a.N] : (long)a.N * a.T;
  bf16* const sPh = (bf16*)(s2 + dq5::RPH);
  bf16* const sPl = (bf16*)(s2 + dq5::RPL);

  struct Unit {
    int u, gc, h, L;
    long tok0;
  };
  auto chunk_s = [&](int gc, int& L, long& tok0) {
    if (a.cu) {
      const int n = sld_i32(a.chunk_idx + 2 * gc);
      if (n < 0) return false;
      const int c = sld_i32(a.chunk_idx + 2 * gc + 1);
      const long b0 = sld_i64(a.cu + n), b1 = sld_i64(a.cu + n + 1);
      tok0 = b0 + (long)c * BT;
      L = min(BT, (int)(b1 - b0) - c * BT);
    } else {
      const int n = gc / a.NT, c = gc - n * a.NT;
      tok0 = (long)n * a.T + (long)c * BT;
      L = min(BT, a.T - c * BT);
    }
    return true;
  };
  auto valid_from = [&](int u) {
    for (; u < nunits; u += gridDim.x) {
      int L;
      long t0;
      if (chunk_s(__builtin_amdgcn_readfirstlane(u / a.H), L, t0)) break;
    }
    return u;
  };
  auto locate = [&](int u) {
    Unit x{u, 0, 0, 1, 0};
    if (u < nunits) {
      x.gc = __builtin_amdgcn_readfirstlane(u / a.H);
      x.h = u - x.gc * a.H;
      chunk_s(x.gc, x.L, x.tok0);
    }
    return x;
  };

  // ---- direct-to-LDS loads
  auto issue_v = [&](char* S, const Unit& x, int vb) {  // 8 per wave
    const int v0 = 32 * vb, l = fresh_lane();
    {
      // h and dS' rows as fp16 (RH, RDH) and their 32 row scales, one copy per wave (RHL, RDHL)
      const long ub = (((long)x.gc * a.H + x.h) * V + v0) * K, sb = ((long)x.gc * a.H + x.h) * V + v0;
      const int r = 4 * w + (l >> 4), p = l & 15;
      const unsigned off = (unsigned)((r * K + 8 * (p ^ (2 * (r & 3)))) * 2), offs = (unsigned)((l & 31) * 4);
      dma16((const bf16*)a.hT + ub, off, S + RH + 1024 * w);
      dma4((const float*)a.hTl + sb, offs, S + RHL + 256 * w);
      dma16((const bf16*)a.dhT + ub, off, S + RDH + 1024 * w);
      dma4((const float*)a.dhTl + sb, offs, S + RDHL + 256 * w);
    }
    const long ub = x.tok0 * rsv + (long)x.h * V + v0;
    {
      const int r = 8 * w + (l >> 3), p = l & 7;
      const unsigned off = (unsigned)((min(r, x.L - 1) * (int)rsv + 4 * (p ^ (r & 7))) * 4);
      dma16(a.U + ub, off, S + RU + 1024 * w);
      dma16(a.dU + ub, off, S + RDU + 1024 * w);
    }
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int j = 2 * w + jj, r = 4 * j + (l >> 4), d = l & 15;
      const unsigned off = (unsigned)((min(r, x.L - 1) * (int)rsv + 8 * ((d >> 2) ^ ((r >> 1) & 3)) + 2 * (d & 3)) * 2);
      dma4((const bf16*)a.dout + ub, off, S + RDO + 256 * j);
    }
  };
  auto issue_qa = [&](char* S, const Unit& x) {  // q_clean (+ g on wave 0)
    const int l = fresh_lane();
    const long ub = x.tok0 * rsk + (long)x.h * K;
    if constexpr (Q32) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int j = 4 * w + jj, r = 2 * j + (l >> 5);
        const unsigned off = (unsigned)((min(r, x.L - 1) * (int)rsk + 4 * (l & 31)) * 4);
        dma16(a.qc32 + ub, off, S + RQ + 1024 * j);
      }
    } else {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int j = 2 * w + jj, r = 4 * j + (l >> 4), p = l & 15;
        const unsigned off = (unsigned)((min(r, x.L - 1) * (int)rsk + 8 * (p ^ (2 * (r & 3)))) * 2);
        dma16((const bf16*)a.qc16 + ub, off, S + 1024 * j);
      }
    }
    // g of the unit's tokens (the last token's past the chunk)
    if (w == 0) dma4(a.gcum + x.tok0 * a.H + x.h, (unsigned)(min(l, x.L - 1) * a.H * 4), (char*)sG);
  };
  auto issue_kp = [&](char* S, const Unit& x) {  // k + P^T: 4 per wave
    const int l = fresh_lane();
    const long ub = x.tok0 * rsk + (long)x.h * K;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int j = 2 * w + jj, r = 4 * j + (l >> 4), p = l & 15;
      const unsigned off = (unsigned)((min(r, x.L - 1) * (int)rsk + 8 * (p ^ (2 * (r & 3)))) * 2);
      dma16((const bf16*)a.k + ub, off, S + dq5::RK + 1024 * j);
    }
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int j = 2 * w + jj, s = 4 * j + (l >> 4), p = l & 15;
      const unsigned off = (unsigned)((s * BT + 4 * (p ^ (s & 15))) * 4);
      dma16(a.PT + ((long)x.gc * a.H + x.h) * (BT * BT), off, S + dq5::RP + 1024 * j);
    }
  };

  f32x16 dQi, dKs, dW, dP;
  float hds;

  // ---- one value piece (as gdn_bwd_dqkw_v4_kernel); `iss` issues this phase's loads between the
  // two 16-value steps (early waves) or after them (the others)
  auto compute_v = [&](const char* S, auto&& iss) {
    const int l = fresh_lane();
    const char* const sch = S + RHL + 256 * w;   // this wave's copy of the h / dS' row scales
    const char* const scd = S + RDHL + 256 * w;
    {
      const int o = 16 * (64 * w + l), r = (64 * w + l) >> 4;
      const i16x8 x1 = *(const i16x8*)(S + RH + o), y1 = *(const i16x8*)(S + RDH + o);
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) d += (float)x1[i] * (float)y1[i];
      hds += d * (*(const float*)(sch + 4 * r) * *(const float*)(scd + 4 * r));
    }
#pragma unroll
    for (int v0 = 0; v0 < 32; v0 += 16) {
      const bf16x8 oa = frag_o(S + RDO, tr, v0, l);
      bf16x8 hb, hbl, db, dbl;
      frag_tr_h16(S + RH, sch, v0, kc, l, hb, hbl);
      frag_tr_h16(S + RDH, scd, v0, kc, l, db, dbl);
      bf16x8 uh, ul, dh, dl;
      frag_u(S + RU, tr, v0, uh, ul, l);
      frag_u(S + RDU, tr, v0, dh, dl, l);
      dQi = mfma(oa, hb, dQi);
      dQi = mfma(oa, hbl, dQi);
      dKs = mfma(uh, db, dKs);
      dKs = mfma(ul, db, dKs);
      dKs = mfma(uh, dbl, dKs);
      dW = mfma(dh, hb, dW);
      dW = mfma(dl, hb, dW);
      dW = mfma(dh, hbl, dW);
      if (dpi == 0 || dpi == 2) {
        dP = mfma(oa, uh, dP);
        dP = mfma(oa, ul, dP);
      } else if (dpi == 1) {
        bf16x8 sh, sl;
        frag_u(S + RU, 0, v0, sh, sl, l);
        dP = mfma(oa, sh, dP);
        dP = mfma(oa, sl, dP);
      }
      if ((v0 == 0) == early) iss();
    }
  };

  // ---- post stage on the q_clean piece Q and the k/P^T piece KP
  auto post = [&](const char* Q, const char* KP, const Unit& x, auto&& iss, auto&& iss_after) {
    const int L = x.L, l = fresh_lane();
    if (early) iss();
    // dP (waves 0, 1, 3): causal and chunk mask, dPs = scale dP Gamma as hi/lo [t][s], dP o P sums
    if (dpi >= 0) {
      const int c = sp + (l & 31);
      const float gcol = sG[c];
      f32x16 e;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r4 = tp + arow(4 * q, l);
        const f32x4 pv = *(const f32x4*)(KP + dq5::RP + off_p(c, r4));  // P[r][c] = P^T[c][r]
        const f32x4 gr = *(const f32x4*)&sG[r4];
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const int i = 4 * q + ii, r = r4 + ii;
          const bool keep = r >= c && r < L;
          const float d = keep ? dP[i] : 0.f;
          const float ev = __expf(gr[ii] - gcol);  // (overflow only where masked)
          const float ps = keep ? d * a.scale * ev : 0.f;
          bf16 hi, lo;
          split2(ps, hi, lo);
          sPh[r * LDP + c] = hi;
          sPl[r * LDP + c] = lo;
          e[i] = d * pv[ii];
        }
      }
      float cs = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) cs += e[i];
      cs += xlane<32>(cs, l);
      if (l < 32) sCP[dpi][l] = cs;
      const float rs = rowsum32(e, l);
      if ((l & 1) == 0) sRP[dpi][arow((l >> 1) & 15, l)] = rs;
    }
    // scale the state parts; dG terms sum_k dQ q_clean and sum_k dK k over this wave's columns
    {
      const int c = kc + (l & 31);
      const float gl = sG[L - 1];
      f32x16 e, f, gv;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 g4 = *(const f32x4*)&sG[tr + arow(4 * q, l)];
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) gv[4 * q + ii] = g4[ii];
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = tr + arow(i, l);
        const float g = gv[i];
        dQi[i] *= a.scale * __expf(g);
        const float qv = Q32 ? *(const float*)(Q + RQ + r * 512 + 4 * c) : (float)*(const bf16*)(Q + off_h(r, c));
        e[i] = dQi[i] * qv;
        dKs[i] *= __expf(gl - g);
        f[i] = dKs[i] * (float)*(const bf16*)(KP + dq5::RK + off_h(r, c));
      }
      const float re = rowsum32(e, l), rf = rowsum32(f, l);
      if ((l & 1) == 0) {
        const int r = tr + arow((l >> 1) & 15, l);
        sRQ[w >> 1][r] = re;
        sRK[w >> 1][r] = rf;
      }
    }
    {
      const float s = wave_sum(hds, l);
      if (l == 0) sHD[w] = s;
    }
    if (!early) iss();
    bar();
    // dq = scale gamma dQi + dPs k (s <= t: the t < 32 half needs s < 32 only)
    {
#pragma unroll
      for (int s0 = 0; s0 < BT; s0 += 16) {
        if (tr == 0 && s0 >= 32) break;
        const bf16x8 kb = frag_tr_h(KP + dq5::RK, s0, kc, l);
        dQi = mfma(frag_rm_l(sPh + tr * LDP + s0, LDP, l), kb, dQi);
        dQi = mfma(frag_rm_l(sPl + tr * LDP + s0, LDP, l), kb, dQi);
      }
      const auto rs = buf_rsrc(a.dq32 + x.tok0 * rsk + (long)x.h * K, (int)(((L - 1) * rsk + K) * 4));
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = tr + arow(i, l);
        const float xq = dQi[i];  // (bit_cast of a vector element reference reads element 0)
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, xq), rs, (int)((r * rsk + kc + (l & 31)) * 4), 0, 0);
      }
    }
    // dk = fac dKs + dPs^T q_clean (i >= j: the j >= 32 half needs i >= 32 only); dw = -dW
    {
      const int c = kc + (l & 31);
#pragma unroll
      for (int i0 = 0; i0 < BT; i0 += 16) {
        if (tr == 32 && i0 < 32) continue;
        const bf16x8 ah = frag32_tr_l(sPh + i0 * LDP + tr, LDP, l), al = frag32_tr_l(sPl + i0 * LDP + tr, LDP, l);
        if constexpr (Q32) {
          bf16x8 bh, bl;
          const int ib = i0 + 8 * (l >> 5);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            bf16 hh, oo;
            split2(*(const float*)(Q + RQ + (ib + e) * 512 + 4 * c), hh, oo);
            bh[e] = hh;
            bl[e] = oo;
          }
          dKs = mfma(ah, bh, dKs);
          dKs = mfma(ah, bl, dKs);
          dKs = mfma(al, bh, dKs);
        } else {
          const bf16x8 bh = frag_tr_h(Q, i0, kc, l);
          dKs = mfma(ah, bh, dKs);
          dKs = mfma(al, bh, dKs);
        }
      }
      // int16 rows with a power-of-two scale per row and 32-column block (this wave's columns): the
      // row maxima by lane exchanges within the half-wave, one scale store per row (lane i of the
      // half-wave stores that of its element i)
      const int bytes = (int)(((L - 1) * rsk + K) * 2);
      const auto rk = buf_rsrc((short*)a.dkp32 + x.tok0 * rsk + (long)x.h * K, bytes);
      const auto rw = buf_rsrc((short*)a.dw32 + x.tok0 * rsk + (long)x.h * K, bytes);
      const f32x16 mk = rowmax32_all(dKs, l), mw = rowmax32_all(dW, l);
      float sk = 0.f, sw = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = tr + arow(i, l), off = (int)((r * rsk + c) * 2);
        const int ek = q16_exp(mk[i]), ew = q16_exp(mw[i]);
        __builtin_amdgcn_raw_buffer_store_b16(q16(dKs[i], ek), rk, off, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b16(q16(-dW[i], ew), rw, off, 0, 0);
        if ((l & 31) == i) {
          sk = ldexpf(1.f, ek);
          sw = ldexpf(1.f, ew);
        }
      }
      if ((l & 31) < 16) {
        const long rsc = (long)a.H * (K / 32);
        const int sbytes = (int)(((L - 1) * rsc + K / 32) * 4);
        const auto rks = buf_rsrc(a.dkp_sc + x.tok0 * rsc + (long)x.h * (K / 32), sbytes);
        const auto rws = buf_rsrc(a.dw_sc + x.tok0 * rsc + (long)x.h * (K / 32), sbytes);
        const int off = (int)(((tr + arow(l & 15, l)) * rsc + kc / 32) * 4);
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, sk), rks, off, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, sw), rws, off, 0, 0);
      }
    }
    bar();
    iss_after();  // the q_clean slot is free
    // decay gradient of token t: (dP o P) row t - column t + dQ o q_clean - dK o k; the last token
    // also takes every dK o k term and e^{G_L} <h, dS'>
    if (w == 0) {
      const int t = l;
      const float term = t < L ? sRK[0][t] + sRK[1][t] + sRK[2][t] + sRK[3][t] : 0.f;
      const float tot = wave_sum(term, l);
      if (t < L) {
        float d = t < 32 ? sRP[0][t] - sCP[0][t] - sCP[1][t]
                         : sRP[1][t - 32] + sRP[2][t - 32] - sCP[2][t - 32];
        d += sRQ[0][t] + sRQ[1][t] + sRQ[2][t] + sRQ[3][t] - term;
        if (t == L - 1) {
          float hsum = 0.f;
#pragma unroll
          for (int ww = 0; ww < 8; ++ww) hsum += sHD[ww];
          d += tot + __expf(sG[L - 1]) * hsum;
        }
        const long gi = (x.tok0 + t) * a.H + x.h;
        a.dgp[gi] = d;
        a.dgp[ntok * a.H + gi] = 0.f;
      }
    }
  };

  // ---- unit loop.  Slots: V0 s0, V1 s1, V2 s2, V3 s0, q_clean s1, k/P^T s2; the next unit's V0
  // is loaded during this unit's post stage, its V1 right after the post stage's products, its V2
  // during its own V0 phase.
  Unit cur = locate(valid_from(blockIdx.x));
  if (cur.u >= nunits) return;
  issue_v(s0, cur, 0);
  issue_v(s1, cur, 1);
  while (true) {
    const Unit nxt = locate(valid_from(cur.u + gridDim.x));
    const bool more = nxt.u < nunits;
    dQi = zero16();
    dKs = zero16();
    dW = zero16();
    dP = zero16();
    hds = 0.f;
    wait_vm<8>();  // V0 (V1 newer; the previous post stage's stores drain with V0)
    bar();
    compute_v(s0, [&] { issue_v(s2, cur, 2); });
    wait_vm<8>();  // V1 (V2 newer)
    bar();
    compute_v(s1, [&] { issue_v(s0, cur, 3); });
    wait_vm<8>();  // V2 (V3 newer)
    bar();
    compute_v(s2, [&] { issue_qa(s1, cur); });
    // V3 (the q_clean piece newer)
    if (w == 0) wait_vm<Q32 ? 5 : 3>();
    else wait_vm<Q32 ? 4 : 2>();
    bar();
    compute_v(s0, [&] { issue_kp(s2, cur); });
    wait_vm<0>();  // q_clean and k/P^T pieces
    bar();
    post(
        s1, s2, cur, [&] { if (more) issue_v(s0, nxt, 0); },
        [&] { if (more) issue_v(s1, nxt, 1); });
    if (!more) break;
    cur = nxt;
  }
}

// ===========================================================================
// launchers (one per kernel so the C ABI can time each launch)
// ===========================================================================
// Compute units of the current device (the persistent kernels launch one workgroup per CU).
static int cu_count() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cache[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

template <int K>
static hipError_t gdn_stage_k(int stage, const GdnArgs& a, int V, hipStream_t st) {
  if (a.NTG == 0) return hipSuccess;
  switch (stage) {
    case kGdnPrep:
      if (K <= 128 && (V == 64 || V == 128)) {
        constexpr int KW = K <= 128 ? K : 128;
        const int grid = min(a.NTG * a.H, cu_count());
        if (V == 128)
          hipLaunchKernelGGL((gdn_prep_v3_kernel<KW, 128>), dim3(grid), dim3(kWalk8), 0, st, a);
        else
          hipLaunchKernelGGL((gdn_prep_v3_kernel<KW, 64>), dim3(grid), dim3(kWalk8), 0, st, a);
      } else {
        hipLaunchKernelGGL(gdn_prep_kernel<K>, dim3(a.NTG, a.H), dim3(kThreads), 0, st, a, V);
      }
      break;
    case kGdnFwdState:
      if (K <= 128) {
        constexpr int KW = K <= 128 ? K : 128;
        const dim3 grid((V / 32) * a.N * a.H);
        const bool s16 = a.snap16 & 1;
        if (a.qc32 && s16)
          hipLaunchKernelGGL((gdn_fwd_state_v3_kernel<KW, true, true>), grid, dim3(kWalk8), 0, st, a, V);
        else if (a.qc32)
          hipLaunchKernelGGL((gdn_fwd_state_v3_kernel<KW, true, false>), grid, dim3(kWalk8), 0, st, a, V);
        else if (s16)
          hipLaunchKernelGGL((gdn_fwd_state_v3_kernel<KW, false, true>), grid, dim3(kWalk8), 0, st, a, V);
        else
          hipLaunchKernelGGL((gdn_fwd_state_v3_kernel<KW, false, false>), grid, dim3(kWalk8), 0, st, a, V);
      } else
        hipLaunchKernelGGL(gdn_fwd_state_kernel<K>, dim3((V / 32) * a.N * a.H), dim3(kThreads), 0, st, a, V);
      break;
    case kGdnFwdO:
      // for K <= 128 the forward walk writes the output itself
      if constexpr (K > 128) {
        if (a.snap16 & 1)
          hipLaunchKernelGGL((gdn_fwd_o_kernel<K, true>), dim3(a.NTG, a.H), dim3(kThreads), 0, st, a, V);
        else
          hipLaunchKernelGGL((gdn_fwd_o_kernel<K, false>), dim3(a.NTG, a.H), dim3(kThreads), 0, st, a, V);
      }
      break;
    case kGdnBwdState:
      if (K <= 128)
      {
        constexpr int KW = K <= 128 ? K : 128;
        const dim3 grid((V / 32) * a.N * a.H);
        const bool s16 = a.snap16 & 2;
        if (a.qc32 && s16)
          hipLaunchKernelGGL((gdn_bwd_state_v3_kernel<KW, true, true>), grid, dim3(kWalk8), 0, st, a, V);
        else if (a.qc32)
          hipLaunchKernelGGL((gdn_bwd_state_v3_kernel<KW, true, false>), grid, dim3(kWalk8), 0, st, a, V);
        else if (s16)
          hipLaunchKernelGGL((gdn_bwd_state_v3_kernel<KW, false, true>), grid, dim3(kWalk8), 0, st, a, V);
        else
          hipLaunchKernelGGL((gdn_bwd_state_v3_kernel<KW, false, false>), grid, dim3(kWalk8), 0, st, a, V);
      }
      else
      {
        if (a.qc32)
          hipLaunchKernelGGL((gdn_bwd_state_kernel<K, true>), dim3((V / 32) * a.N * a.H), dim3(kThreads), 0, st, a, V);
        else
          hipLaunchKernelGGL((gdn_bwd_state_kernel<K, false>), dim3((V / 32) * a.N * a.H), dim3(kThreads), 0, st, a, V);
      }
      break;
    case kGdnBwdDqkw:
      if (K == 128 && V == 128) {
        const int grid = min(a.NTG * a.H, cu_count());
        if (a.qc32)
          hipLaunchKernelGGL(gdn_bwd_dqkw_v5_kernel<true>, dim3(grid), dim3(kWalk8), 0, st, a);
        else
          hipLaunchKernelGGL(gdn_bwd_dqkw_v5_kernel<false>, dim3(grid), dim3(kWalk8), 0, st, a);
      } else if (K == 128 && V == 64 && a.qc32) {
        hipLaunchKernelGGL(gdn_bwd_dqkw_v4_kernel<64>, dim3(min(a.NTG * a.H, cu_count())), dim3(kWalk8), 0, st, a);
      } else if (K == 128)
        hipLaunchKernelGGL(gdn_bwd_dqkw_v3_kernel<128>, dim3(1, a.NTG, a.H), dim3(kWalk8), 0, st, a, V);
      else {
        const dim3 grid((K / 64) * a.NTG * a.H);
        switch (a.snap16 & 3) {
          case 3: hipLaunchKernelGGL((gdn_bwd_dqkw_v2_kernel<K, true, true>), grid, dim3(kThreads), 0, st, a, V); break;
          case 1: hipLaunchKernelGGL((gdn_bwd_dqkw_v2_kernel<K, true, false>), grid, dim3(kThreads), 0, st, a, V); break;
          case 2: hipLaunchKernelGGL((gdn_bwd_dqkw_v2_kernel<K, false, true>), grid, dim3(kThreads), 0, st, a, V); break;
          default: hipLaunchKernelGGL((gdn_bwd_dqkw_v2_kernel<K, false, false>), grid, dim3(kThreads), 0, st, a, V);
        }
      }
      break;
    case kGdnBwdWy:
      if (K <= 128 && (V == 64 || V == 128)) {
        constexpr int KW = K <= 128 ? K : 128;
        const int grid = min(a.NTG * a.H, cu_count());
        if (V == 128)
          hipLaunchKernelGGL((gdn_bwd_wy_v3_kernel<KW, 128>), dim3(grid), dim3(kWalk8), 0, st, a);
        else
          hipLaunchKernelGGL((gdn_bwd_wy_v3_kernel<KW, 64>), dim3(grid), dim3(kWalk8), 0, st, a);
      } else {
        hipLaunchKernelGGL(gdn_bwd_wy_v2_kernel<K>, dim3(a.NTG, a.H), dim3(kThreads), 0, st, a, V);
      }
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_gdn_stage(int stage, const GdnArgs& a, int K, int V, hipStream_t st) {
  switch (K) {
    case 64: return gdn_stage_k<64>(stage, a, V, st);
    case 128: return gdn_stage_k<128>(stage, a, V, st);
    case 256: return gdn_stage_k<256>(stage, a, V, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ccq
