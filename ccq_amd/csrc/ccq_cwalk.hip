// CCQ read-side cleaning operator on gfx950: column walks (forward and backward) for K = 32 and
// K = 256 (K = 64 and 128 run as segment walks, ccq_cseg.hip).
//
// Mathematics (per sequence and head; reference ccq/ops/common/fused_read.py:11-25):
//   C_t = h_0 + sum_{j<=t} k_j k_j^T     m_t = m_0 + sum_{j<=t} k_j
//   z_t = C_t^T q_t     s_t = m_t . q_t     corr_t = z_t/pos_t - s_t m_t/pos_t^2
//   q_clean_t = q_t - lambda_t corr_t
// Backward (closed form, fused_read.py:18-25), dz_t = -lambda_t dqc_t / pos_t:
//   dlambda_t = -dqc_t . corr_t      ds_t = lambda_t (dqc_t . m_t)/pos_t^2
//   dm_t = lambda_t s_t dqc_t/pos_t^2 + ds_t q_t  (= -(s_t/pos_t) dz_t + ds_t q_t)
//   dq_t = dqc_t + ds_t m_t + C_t dz_t (+ gate: dlogit_t w, dlogit_t = dlambda_t lambda_t (1-lambda_t))
//   dk_j = E_j k_j + sum_{t>=j} dm_t + dm_T,  E_j = sum_{t>=j} (q_t dz_t^T + dz_t q_t^T) + dC_T + dC_T^T
//   dC_0 = sum_t q_t dz_t^T + dC_T,   dm_0 = sum_t dm_t + dm_T
// C is symmetric (h_0 is taken as symmetric: it is a sum of k k^T in every caller), so a column
// slice of C is also a row slice.
//
// Layout of the work: a workgroup owns 32 columns of the K x K state for one (sequence, head) and
// walks the sequence in CB-token chunks, keeping its state slice in fp32 registers -- no state goes
// to HBM.  Per chunk (Q, K, dZ its rows; M the causal mask incl. the diagonal):
//   forward   Z[:, cols] = Q C_prev[:, cols] + ((Q K^T) o M) K[:, cols],  C += K^T K[:, cols]
//   dq walk   dQ[:, cols] = dZ C_prev[:, cols] + ((dZ K^T) o M) K[:, cols] + ...  (forward order)
//   dk walk   dK[:, cols] = K E[:, cols] + ((dZ K^T) o M)^T Q[:, cols] + ((Q K^T) o M)^T dZ[:, cols]
//             + suffix sums of dm, with E = G + G^T walked in reverse (G += Q^T dZ)
// The per-chunk score blocks are recomputed by each column workgroup of a head (a CB x CB x K
// product).  fp32 operands (states, scores, dz) enter the MFMAs as hi/lo bf16 pairs written once
// per chunk into LDS, so every product keeps ~16 significant bits.  Waves 0..NB-1 produce the
// output rows, the other waves own the state slice (row tiles round-robin).
//
// Kernels:
//   cw_fwd   forward walk: q_clean, z (kept for the backward), s_t, chunk-start key sums, C_T, m_T
//   cw_rows  backward, chunk-parallel: per-token scalars (-lambda/pos, ds, dlambda or dlogit,
//            -s/pos), dlambda, gate partials
//   cw_dq    backward forward-walk: dq
//   cw_dk    backward reverse-walk: dk, dC_0, dm_0
#include "ccq_tile.h"
#include "ccq_walk_args.h"

namespace ccq {

namespace {

template <int K>
struct Walk {
  static constexpr int CB = walk_chunk(K);          // tokens per chunk
  static constexpr int NB = CB / 32;                // 32-row blocks per chunk (= output waves)
  static constexpr int NSW = 4 - NB;                // waves that own the state slice
  static constexpr int NRT = K / 32;                // 32-row tiles of the state slice
  static constexpr int TPW = (NRT + NSW - 1) / NSW;  // state tiles per state wave
  static constexpr int LDK = K + 8, LDA = CB + 8;   // LDS leading dimensions (bf16 elements)
  static constexpr int NBLK = NB * (NB + 1) / 2;    // causal 32 x 32 score blocks per chunk
};

__device__ __forceinline__ float cw_pos(int t, int off) {
  const float p = (float)(t + 1 + off);
  return p < 1.f ? 1.f : p;
}

__device__ __forceinline__ bf16x8 ones8() {
  bf16x8 v;
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (bf16)1.f;
  return v;
}

// Score block b of a chunk as (row block, column block) with column block <= row block:
// b = 0 -> (0, 0), 1 -> (1, 0), 2 -> (1, 1).
__device__ __forceinline__ int blk_row(int b) { return b == 0 ? 0 : 1; }
__device__ __forceinline__ int blk_col(int b) { return b == 2 ? 1 : 0; }

// Offset (in rows) of accumulator element i from the lane's first row (acc_row(0)).
__device__ __forceinline__ constexpr int acc_drow(int i) { return 8 * (i >> 2) + (i & 3); }

// Store a lane's 16 accumulator values to rows base + acc_drow(i) * rs of an fp32 or bf16 tensor;
// rows at or beyond `nrows` (counted from the tile's first row, r0 = this lane's first row) are
// skipped.  Full tiles take a branch-free path.
__device__ __forceinline__ void store16(float* p32, bf16* p16, long base, long rs, const float (&v)[16], int r0,
                                        int nrows) {
  if (r0 + 27 < nrows) {
    if (p32) {
#pragma unroll
      for (int i = 0; i < 16; ++i) p32[base + acc_drow(i) * rs] = v[i];
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) gmem(p16)[base + acc_drow(i) * rs] = (bf16)v[i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (r0 + acc_drow(i) < nrows) {
        if (p32) p32[base + acc_drow(i) * rs] = v[i];
        else gmem(p16)[base + acc_drow(i) * rs] = (bf16)v[i];
      }
    }
  }
}

// Load a lane's 16 values, rows r0 + acc_drow(i) of a chunk whose row 0 is at base (rows at or beyond
// nrows >= 1 read row 0 instead: always in bounds, value unused), of an fp32 or bf16 tensor.
__device__ __forceinline__ void load16(const float* p32, const bf16* p16, long base, long rs, float (&v)[16], int r0,
                                       int nrows) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const long e = base + (long)(r0 + acc_drow(i) < nrows ? r0 + acc_drow(i) : 0) * rs;
    v[i] = p32 ? p32[e] : (float)gmem(p16)[e];
  }
}

// One walk: (sequence, head, 32-column tile, time segment).  Chunks [cb, ce) of the sequence's nc
// chunks; with one segment that is the whole sequence.  Segments are whole 64-token blocks (the
// blocks of the segment sums, ccq_cseg.hip): nc64 blocks cut into pieces of ceil(nc64 / nseg).
struct WalkUnit {
  int unit, ct, c0, seg, nseg, h, n, len, nc, cb, ce, gc0;
  long bos, hb, rs;
};

// Workgroup -> (sequence, head, 32-column tile, segment); the workgroups of one (sequence, head)
// share an XCD.
template <int K>
__device__ __forceinline__ WalkUnit walk_unit(const WalkArgs& a) {
  WalkUnit u;
  u.nseg = a.segD ? a.nseg : 1;
  int sub;
  xcd_map(blockIdx.x, (K / 32) * u.nseg, a.N * a.H, u.unit, sub);
  u.ct = sub % (K / 32);
  u.seg = sub / (K / 32);
  u.n = u.unit / a.H;
  u.h = u.unit % a.H;
  u.c0 = u.ct * 32;
  seq_bounds(a.cu, u.n, a.T, u.bos, u.len);
  u.nc = (u.len + Walk<K>::CB - 1) / Walk<K>::CB;
  {
    constexpr int R = 64 / Walk<K>::CB;  // walk chunks per 64-token block
    const int nb = (u.len + 63) / 64, per = (nb + u.nseg - 1) / u.nseg;
    const int b0 = min(nb, u.seg * per), b1 = min(nb, b0 + per);
    u.cb = min(u.nc, b0 * R);
    u.ce = min(u.nc, b1 * R);
  }
  u.gc0 = a.cu ? a.chunk_off[u.n] : u.n * a.NT;
  u.rs = (long)a.H * K;
  u.hb = (u.bos * a.H + u.h) * (long)K;  // element (t, c) of the sequence: hb + t * rs + c
  return u;
}

// dz_t = F_t dqc_t for a CB x K chunk (F_t = -lambda_t / pos_t, the first of the four row scalars),
// prefetched by NTHR threads (local index lt) and written to LDS as a hi/lo bf16 pair, row-major.
// Thread lt covers rows lt/8 + RP m (RP = NTHR/8) and columns 4 (lt%8) + 32 s: eight lanes read one
// contiguous 128-byte piece of a row, and a thread needs the row scalar of only CB/RP rows.  The
// upstream gradient is fp32 or bf16 (four elements per slot).  Rows at or beyond nvalid read row 0
// (always valid) and are zeroed when stored.
template <int K, int CB, int NTHR>
struct PrefetchDzRows {
  static constexpr int RP = NTHR / 8, RPASS = (CB + RP - 1) / RP, CPASS = K / 32, N = RPASS * CPASS;
  f32x4 v[N];
  float f[RPASS];
  __device__ __forceinline__ void load(const float* g32, const bf16* g16, long gstride, const float* sc,
                                       long sstride, int nvalid, int lt) {
    const int r0 = lt >> 3, c0 = (lt & 7) * 4;
#pragma unroll
    for (int m = 0; m < RPASS; ++m) {
      const int r = r0 + RP * m;
      const long rr = (r < nvalid && r < CB) ? r : 0;
      f[m] = sc[rr * sstride];
#pragma unroll
      for (int s = 0; s < CPASS; ++s) {
        const long e = rr * gstride + c0 + 32 * s;
        if (g32) {
          v[m * CPASS + s] = *(const f32x4*)(g32 + e);
        } else {
          const bf16x4 b = *(const bf16x4*)(g16 + e);
#pragma unroll
          for (int i = 0; i < 4; ++i) v[m * CPASS + s][i] = (float)b[i];
        }
      }
    }
  }
  __device__ __forceinline__ void store(bf16* hi, bf16* lo, int ld, int nvalid, int lt) const {
    const int r0 = lt >> 3, c0 = (lt & 7) * 4;
#pragma unroll
    for (int m = 0; m < RPASS; ++m) {
      const int r = r0 + RP * m;
      if (CB % RP != 0 && r >= CB) continue;
      const float fm = (r < nvalid) ? f[m] : 0.f;
#pragma unroll
      for (int s = 0; s < CPASS; ++s) {
        bf16x4 vh, vl;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          bf16 a, b;
          split2(v[m * CPASS + s][i] * fm, a, b);
          vh[i] = a;
          vl[i] = b;
        }
        *(bf16x4*)(hi + r * ld + c0 + 32 * s) = vh;
        *(bf16x4*)(lo + r * ld + c0 + 32 * s) = vl;
      }
    }
  }
};

// Register prefetch of a ROWS x D bf16 tile by NTHR threads (local index lt), one chunk ahead.
// Rows at or beyond nvalid are loaded from row 0 (always valid) and zeroed when stored, so the loads
// carry no branches.
template <int D, int ROWS, int NTHR>
struct PrefetchRows {
  static constexpr int VPR = D / 8, TOT = ROWS * VPR;
  static constexpr int N = (TOT + NTHR - 1) / NTHR;
  bf16x8 v[N];
  __device__ __forceinline__ void load(const bf16* g, long gstride, int nvalid, int lt) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = min(lt + j * NTHR, TOT - 1);
      const int r = idx / VPR, c = (idx % VPR) * 8;
      v[j] = *(const bf16x8*)(g + (long)(r < nvalid ? r : 0) * gstride + c);
    }
  }
  __device__ __forceinline__ void store(bf16* dst, int ld, int nvalid, int lt) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = lt + j * NTHR;
      if (TOT % NTHR != 0 && idx >= TOT) continue;
      const int r = idx / VPR, c = (idx % VPR) * 8;
      bf16x8 x = v[j];
      if (r >= nvalid) x = bf16x8{};
      *(bf16x8*)(dst + r * ld + c) = x;
    }
  }
};

// Initial state slice of a state wave: tile j = rows (sw + NSW j) * 32 .. +31, columns c0 .. c0+31 of
// a [K, K] fp32 matrix at p (nullable -> zeros); `transposed` reads p[c][r] instead.
template <int K>
__device__ __forceinline__ void load_slice(f32x16 (&S)[Walk<K>::TPW], const float* p, int sw, int c0,
                                           bool transposed) {
#pragma unroll
  for (int j = 0; j < Walk<K>::TPW; ++j) {
    const int rt = sw + Walk<K>::NSW * j;
    S[j] = zero16();
    if (p && sw >= 0 && rt < Walk<K>::NRT) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = rt * 32 + acc_row(i), c = c0 + acc_col();
        S[j][i] = transposed ? p[(long)c * K + r] : p[(long)r * K + c];
      }
    }
  }
}

template <int K>
__device__ __forceinline__ void store_slice(const f32x16 (&S)[Walk<K>::TPW], float* p, int sw, int c0) {
#pragma unroll
  for (int j = 0; j < Walk<K>::TPW; ++j) {
    const int rt = sw + Walk<K>::NSW * j;
    if (sw >= 0 && rt < Walk<K>::NRT) {
#pragma unroll
      for (int i = 0; i < 16; ++i) p[(long)(rt * 32 + acc_row(i)) * K + c0 + acc_col()] = S[j][i];
    }
  }
}

// Add the segment totals tot[unit][s] (fp32 [K, K] each) for s in [s0, s1) to a state slice
// (tiles as load_slice), optionally with their transposes.
template <int K>
__device__ __forceinline__ void add_seg_slice(f32x16 (&S)[Walk<K>::TPW], const float* tot, long unit, int nseg, int s0,
                                              int s1, int sw, int c0, bool with_transpose) {
  for (int s = s0; s < s1; ++s) {
    const float* p = tot + ((long)unit * nseg + s) * K * K;
#pragma unroll
    for (int j = 0; j < Walk<K>::TPW; ++j) {
      const int rt = sw + Walk<K>::NSW * j;
      if (sw >= 0 && rt < Walk<K>::NRT) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int r = rt * 32 + acc_row(i), c = c0 + acc_col();
          S[j][i] += p[(long)r * K + c] + (with_transpose ? p[(long)c * K + r] : 0.f);
        }
      }
    }
  }
}

}  // namespace

// ===========================================================================
// cw_fwd: grid N*H*(K/32)*nseg.  Roles: output waves (0..NB-1) compute the chunk's rows and do every
// global store; state waves (NB..3) own the state slice and do every global load (one chunk ahead),
// so a wave that stores never waits for a load and vice versa.
//   stage    state waves: Q, K, lambda, C[:, cols] (hi/lo), m_prev (fp32 + hi/lo) into LDS
//   phase 1  waves 0..NBLK-1: score blocks; wave 3: row products Q [m_hi m_lo w_hi w_lo] on the
//            MFMA (m_prev . q_t and the gate logit) and 1/pos_t
//   phase 2  output waves: Z, running key sums, q_clean; state waves: C and key-sum update
// ===========================================================================
template <int K>
__global__ __launch_bounds__(kThreads) void cw_fwd_kernel(const WalkArgs a) {
  using W = Walk<K>;
  constexpr int CB = W::CB, NB = W::NB, NSW = W::NSW, NRT = W::NRT, TPW = W::TPW, LDK = W::LDK, LDA = W::LDA;
  constexpr int NLT = NSW * 64;  // loader threads
  __shared__ __attribute__((aligned(16))) bf16 sQ[2][CB * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sK[2][CB * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sCh[2][32 * LDK];  // C[:, cols] as [col][row], hi
  __shared__ __attribute__((aligned(16))) bf16 sCl[2][32 * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sAh[CB * LDA];     // scores A[t][s] (s <= t), hi
  __shared__ __attribute__((aligned(16))) bf16 sAl[CB * LDA];
  __shared__ __attribute__((aligned(16))) bf16 sMW[2][4 * LDK];   // rows m_hi, m_lo, w_hi, w_lo
  __shared__ __attribute__((aligned(16))) float sM[2][K];         // key sum before the chunk
  __shared__ __attribute__((aligned(16))) float sLam[2][CB];
  __shared__ __attribute__((aligned(16))) float sS[CB];           // m_prev . q_t
  __shared__ __attribute__((aligned(16))) float sIp[CB];          // 1 / pos_t
  __shared__ __attribute__((aligned(16))) float sRA[2][CB];       // row sums of the score blocks
  __shared__ __attribute__((aligned(16))) float sRD[32 * (CB + 4)];  // row products, [column][row]

  const int tid = threadIdx.x, w = wave_id(), l = lane_id();
  const WalkUnit u = walk_unit<K>(a);
  const bool mean = a.subtract_mean != 0, gate = a.gate_w != nullptr;
  const int sw = w - NB;       // state-wave index (< 0 on output waves)
  const int lt = tid - NB * 64;  // loader-thread index (state waves)
  const float gbias = gate ? a.gate_b[u.h] : 0.f;

  // state at the segment start: h_0 (+ the earlier segments' K^T K and key sums)
  f32x16 C[TPW], Mk[TPW];
  load_slice<K>(C, a.h0 ? a.h0 + (long)u.unit * K * K : nullptr, sw, u.c0, false);
  if (u.seg > 0) add_seg_slice<K>(C, a.segD, u.unit, u.nseg, 0, u.seg, sw, u.c0, false);
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int rt = sw + NSW * j;
    Mk[j] = zero16();
    if (mean && sw >= 0 && rt < NRT) {
      float m = a.m0 ? a.m0[(long)u.unit * K + rt * 32 + acc_col()] : 0.f;
      for (int s2 = 0; s2 < u.seg; ++s2) m += a.segM[((long)u.unit * u.nseg + s2) * K + rt * 32 + acc_col()];
#pragma unroll
      for (int i = 0; i < 16; ++i) Mk[j][i] = m;
    }
  }
  for (int c = tid; c < K; c += kThreads) {
    bf16 hh = (bf16)0.f, ll = (bf16)0.f;
    if (gate) split2(a.gate_w[(long)u.h * K + c], hh, ll);
    sMW[0][2 * LDK + c] = hh;
    sMW[0][3 * LDK + c] = ll;
    sMW[1][2 * LDK + c] = hh;
    sMW[1][3 * LDK + c] = ll;
  }

  PrefetchRows<K, CB, NLT> pq, pk;
  float plam = 0.f;
  auto issue = [&](int c) {
    const int L = min(CB, u.len - c * CB);
    const long off = u.hb + (long)c * CB * u.rs;
    pq.load((const bf16*)a.q + off, u.rs, L, lt);
    pk.load((const bf16*)a.k + off, u.rs, L, lt);
    if (!gate && lt < CB) plam = a.lam[(u.bos + (long)c * CB + min(lt, L - 1)) * a.H + u.h];
  };
  if (sw >= 0 && u.cb < u.ce) issue(u.cb);

  for (int c = u.cb; c < u.ce; ++c) {
    const int b = c & 1, t0 = c * CB, L = min(CB, u.len - t0);
    bf16* Q = sQ[b];
    bf16* Kc = sK[b];
    // ---- stage (state waves)
    if (sw >= 0) {
      pq.store(Q, LDK, L, lt);
      pk.store(Kc, LDK, L, lt);
      if (!gate && lt < CB) sLam[b][lt] = (lt < L) ? plam : 0.f;
#pragma unroll
      for (int j = 0; j < TPW; ++j) {
        const int rt = sw + NSW * j;
        if (rt < NRT) {
          acc_to_lds_t(C[j], sCh[b], sCl[b], LDK, rt * 32);
          if (l < 32) {
            const float m = Mk[j][0];
            bf16 hh, ll;
            split2(m, hh, ll);
            sM[b][rt * 32 + l] = m;
            sMW[b][rt * 32 + l] = hh;
            sMW[b][LDK + rt * 32 + l] = ll;
          }
        }
      }
    }
    __syncthreads();

    // ---- phase 1
    if (sw >= 0 && c + 1 < u.ce) issue(c + 1);
    if (w < W::NBLK) {
      // score block A^T = K_J Q_I^T: element (s, t) = k_s . q_t, kept for s <= t
      const int I = blk_row(w), J = blk_col(w);
      f32x16 acc = zero16();
      mma_rr(acc, Kc + J * 32 * LDK, LDK, Q + I * 32 * LDK, LDK, K);
      float rsum = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (32 * J + acc_row(i) > 32 * I + acc_col()) acc[i] = 0.f;
        rsum += acc[i];
      }
      acc_to_lds_t(acc, sAh + I * 32 * LDA, sAl + I * 32 * LDA, LDA, 32 * J);
      rsum += __shfl_xor(rsum, 32);
      if (l < 32) sRA[J][32 * I + l] = rsum;
    } else if (w == 3) {
      // columns 0..3 of Q [m_hi m_lo w_hi w_lo] (other columns zero): m_prev . q_t = col0 + col1,
      // gate logit = col2 + col3.  All 32 columns go to LDS ([column][row]); one lane per row then
      // finishes the row scalars.
      constexpr int LDR = CB + 4;
      const int n = l & 31;
      const bf16* mw = sMW[b] + min(n, 3) * LDK + ((l >> 5) << 3);
#pragma unroll
      for (int I = 0; I < NB; ++I) {
        f32x16 acc = zero16();
#pragma unroll
        for (int k0 = 0; k0 < K; k0 += 16) {
          bf16x8 bf = *(const bf16x8*)(mw + k0);
          if (n >= 4) bf = bf16x8{};
          acc = mfma(frag_rm(Q + I * 32 * LDK + k0, LDK), bf, acc);
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          f32x4 v;
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = acc[4 * g + i];
          *(f32x4*)(sRD + n * LDR + 32 * I + acc_row(4 * g)) = v;
        }
      }
      const int t = l & (CB - 1);
      const float mq = sRD[t] + sRD[LDR + t];
      const float lg = sRD[2 * LDR + t] + sRD[3 * LDR + t];
      if (l < CB) {
        sS[t] = mean ? mq : 0.f;
        sIp[t] = __builtin_amdgcn_rcpf(cw_pos(t0 + t, a.pos_off));
        if (gate) sLam[b][t] = (t < L) ? __builtin_amdgcn_rcpf(1.f + __expf(-(lg + gbias))) : 0.f;
      }
    }
    __syncthreads();

    // ---- phase 2
    if (w < NB) {
      const int I = w;
      f32x16 zacc = zero16(), cum = zero16();
      const bf16* Qr = Q + I * 32 * LDK;
#pragma unroll 4
      for (int k0 = 0; k0 < K; k0 += 16) {
        const bf16x8 qf = frag_rm(Qr + k0, LDK);
        zacc = mfma(qf, frag_rm(sCh[b] + k0, LDK), zacc);
        zacc = mfma(qf, frag_rm(sCl[b] + k0, LDK), zacc);
      }
      for (int s0 = 0; s0 < 32 * (I + 1); s0 += 16) {
        const bf16x8 kf = frag32_tr(Kc + s0 * LDK + u.c0, LDK);
        zacc = mfma(frag_rm(sAh + I * 32 * LDA + s0, LDA), kf, zacc);
        zacc = mfma(frag_rm(sAl + I * 32 * LDA + s0, LDA), kf, zacc);
        if (mean) cum = mfma(frag_tril_ones(32 * I, s0), kf, cum);
      }
      const int cc = acc_col();
      const float mc = sM[b][u.c0 + cc];
      // row scalars of this lane's 16 rows (four groups of four consecutive rows)
      float sv[16], ipv[16], lmv[16];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int t4 = 32 * I + acc_row(4 * g);
        const f32x4 s0 = *(const f32x4*)(sS + t4), r0 = *(const f32x4*)(sRA[0] + t4);
        const f32x4 r1 = (NB == 2 && I == 1) ? *(const f32x4*)(sRA[1] + t4) : f32x4{};
        const f32x4 ip4 = *(const f32x4*)(sIp + t4), l4 = *(const f32x4*)(sLam[b] + t4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sv[4 * g + i] = mean ? s0[i] + r0[i] + r1[i] : 0.f;
          ipv[4 * g + i] = ip4[i];
          lmv[4 * g + i] = l4[i];
        }
      }
      const int r0 = 32 * I + acc_row(0);
      const long rowbase = u.hb + (long)(t0 + r0) * u.rs + u.c0 + cc;
      float qv[16], zo[16], qo[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) qv[i] = (float)Q[(r0 + acc_drow(i)) * LDK + u.c0 + cc];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float ip = ipv[i];
        zo[i] = zacc[i];
        qo[i] = qv[i] - lmv[i] * (zacc[i] * ip - sv[i] * ip * ip * (mc + cum[i]));
      }
      store16(a.z, nullptr, rowbase, u.rs, zo, r0, L);
      store16(a.qc32, (bf16*)a.qc, rowbase, u.rs, qo, r0, L);
      if (u.ct == 0 && cc == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int t = 32 * I + acc_row(i);
          if (t < L) {
            const long ti = (u.bos + t0 + t) * a.H + u.h;
            a.srow[ti] = sv[i];
            if (gate && a.lam_out) a.lam_out[ti] = lmv[i];
          }
        }
      }
      if (mean && u.ct == 0)
        for (int i = tid; i < K; i += NB * 64) a.mpre[((long)(u.gc0 + c) * a.H + u.h) * K + i] = sM[b][i];
    } else {
      bf16x8 kc[CB / 16];
#pragma unroll
      for (int s = 0; s < CB / 16; ++s) kc[s] = frag32_tr(Kc + s * 16 * LDK + u.c0, LDK);
#pragma unroll
      for (int j = 0; j < TPW; ++j) {
        const int rt = sw + NSW * j;
        if (rt < NRT) {
#pragma unroll
          for (int s = 0; s < CB / 16; ++s) {
            const bf16x8 kr = frag32_tr(Kc + s * 16 * LDK + rt * 32, LDK);  // (r, s) = k_s[rt*32 + r]
            C[j] = mfma(kr, kc[s], C[j]);
            if (mean) Mk[j] = mfma(ones8(), kr, Mk[j]);
          }
        }
      }
    }
  }

  const bool last = u.seg == u.nseg - 1;
  if (last && a.h_fin) store_slice<K>(C, a.h_fin + (long)u.unit * K * K, sw, u.c0);
  if (last && mean && u.ct == 0 && a.m_fin && sw >= 0 && l < 32) {
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int rt = sw + NSW * j;
      if (rt < NRT) a.m_fin[(long)u.unit * K + rt * 32 + l] = Mk[j][0];
    }
  }
}

// ===========================================================================
// cw_rows: grid NTG*H, one workgroup per (chunk, head); HBM-bound.  Every thread issues all of its
// loads up front:
//   key sums   m_t = m_prev + prefix of k over the chunk: column c = tid % K, row segment
//              seg = tid / K (NSEG = 256 / K segments of RPS rows); local prefixes in LDS, segment
//              offsets (m_prev + totals of earlier segments) applied when read
//   row dots   thread = (row t = tid / TPR, column part): dqc . z_t and dqc . m_t
//   scalars    -lambda/pos, ds, dlambda (or dlogit), -s/pos per token; dlambda
//   columns    per-chunk sums over t of dm_t = (lambda_t s_t/pos_t^2) dqc_t + ds_t q_t (the dk walk's
//              carry) and the gate partials dW = sum_t dlogit_t q_t, db = sum_t dlogit_t (segment
//              split as the key sums)
// ===========================================================================
template <int K>
__global__ __launch_bounds__(kThreads) void cw_rows_kernel(const WalkArgs a) {
  constexpr int CB = Walk<K>::CB, TPR = kThreads / CB, PER = K / TPR, LDM = K + 4;
  constexpr int NSEG = kThreads / K > 0 ? kThreads / K : 1, RPS = CB / NSEG;
  __shared__ __attribute__((aligned(16))) float sMt[CB * LDM];  // local prefixes of k
  __shared__ float sOff[NSEG][K];                                // segment offsets of m
  __shared__ float sG[CB];                                       // dlogit_t (gate)
  __shared__ float sW[NSEG][K];                                  // gate partials per segment
  __shared__ float sD[NSEG][K];                                  // dm column sums per segment
  const int gc = blockIdx.x / a.H, h = blockIdx.x % a.H, tid = threadIdx.x;
  const bool gate = a.gate_w != nullptr, mean = a.subtract_mean != 0;
  int n, c;
  if (a.cu) {
    n = a.chunk_idx[2 * gc];
    c = a.chunk_idx[2 * gc + 1];
  } else {
    n = gc / a.NT;
    c = gc % a.NT;
  }
  float* dwp = gate ? a.dw_part + ((long)gc * a.H + h) * K : nullptr;
  if (n < 0) {  // padding entry of a varlen launch
    if (gate) {
      for (int i = tid; i < K; i += kThreads) dwp[i] = 0.f;
      if (tid == 0) a.db_part[(long)gc * a.H + h] = 0.f;
    }
    return;
  }
  long bos;
  int len;
  seq_bounds(a.cu, n, a.T, bos, len);
  const int t0 = c * CB, L = min(CB, len - t0);
  const long rs = (long)a.H * K, hb = (bos * a.H + h) * (long)K + (long)t0 * rs;
  const int col = tid % K, seg = tid / K;  // column role (tid < NSEG * K)

  // row-dot role: loads first
  const int t = tid / TPR, part = tid % TPR;
  const long e0 = hb + (long)(t < L ? t : 0) * rs + part * PER;
  f32x4 zv[PER / 4], gv[PER / 4];
  bf16x8 qv8[PER / 8], kv8[PER / 8];
  if (mean || gate) {
#pragma unroll
    for (int j = 0; j < PER / 8; ++j) qv8[j] = *(const bf16x8*)((const bf16*)a.q + e0 + 8 * j);
  }
  if (mean) {
#pragma unroll
    for (int j = 0; j < PER / 8; ++j) kv8[j] = *(const bf16x8*)((const bf16*)a.k + e0 + 8 * j);
  }
#pragma unroll
  for (int j = 0; j < PER / 4; ++j) {
    zv[j] = *(const f32x4*)(a.z + e0 + 4 * j);
    if (a.dqc32) {
      gv[j] = *(const f32x4*)(a.dqc32 + e0 + 4 * j);
    } else {
      const bf16x4 bv = *(const bf16x4*)((const bf16*)a.dqc16 + e0 + 4 * j);
#pragma unroll
      for (int i = 0; i < 4; ++i) gv[j][i] = (float)bv[i];
    }
  }
  if (mean) {
    // k rows into LDS (zero past the chunk), then local column prefixes over each row segment
#pragma unroll
    for (int j = 0; j < PER / 8; ++j) {
      f32x4 k0, k1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        k0[i] = t < L ? (float)kv8[j][i] : 0.f;
        k1[i] = t < L ? (float)kv8[j][4 + i] : 0.f;
      }
      *(f32x4*)(sMt + t * LDM + part * PER + 8 * j) = k0;
      *(f32x4*)(sMt + t * LDM + part * PER + 8 * j + 4) = k1;
    }
    __syncthreads();
    if (tid < NSEG * K) {
      float acc = 0.f;
#pragma unroll
      for (int r = 0; r < RPS; ++r) {
        float* m = sMt + (seg * RPS + r) * LDM + col;
        acc += *m;
        *m = acc;
      }
      sOff[seg][col] = acc;  // segment total for now
    }
  }
  __syncthreads();
  if (mean && tid < K) {
    float off = a.mpre[((long)gc * a.H + h) * K + tid];
    for (int sg = 0; sg < NSEG; ++sg) {
      const float tot = sOff[sg][tid];
      sOff[sg][tid] = off;
      off += tot;
    }
  }
  __syncthreads();

  float dzd = 0.f, dmd = 0.f;
  const int sgt = t / RPS;
#pragma unroll
  for (int j = 0; j < PER / 4; ++j) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dzd += gv[j][i] * zv[j][i];
      if (mean) {
        const int cc = part * PER + 4 * j + i;
        dmd += gv[j][i] * (sMt[t * LDM + cc] + sOff[sgt][cc]);
      }
    }
  }
  dzd = group_sum(dzd, TPR);
  dmd = group_sum(dmd, TPR);
  float g = 0.f, am = 0.f, ds = 0.f;
  if (t < L) {
    const long ti = (bos + t0 + t) * a.H + h;
    const float lam = a.lam_used[ti];
    const float p = cw_pos(t0 + t, a.pos_off);
    const float s = mean ? a.srow[ti] : 0.f;
    const float dcorr = dzd / p - (mean ? s * dmd / (p * p) : 0.f);  // dqc . corr
    const float dlam = -dcorr;
    g = gate ? dlam * lam * (1.f - lam) : dlam;
    ds = mean ? lam * dmd / (p * p) : 0.f;
    am = mean ? lam * s / (p * p) : 0.f;
    if (part == 0) {
      f32x4 o;
      o[0] = -lam / p;
      o[1] = ds;
      o[2] = g;
      o[3] = -s / p;
      *(f32x4*)(a.sc + ti * 4) = o;
      if (!gate && a.dlam) a.dlam[ti] = dlam;
    }
    if (a.dzh) {
      // dz_t = F_t dqc_t for this thread's columns, as a hi/lo bf16 pair
      const float F = -lam / p;
#pragma unroll
      for (int j = 0; j < PER / 8; ++j) {
        bf16x8 vh, vl;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          bf16 x, y;
          split2(F * gv[2 * j + i / 4][i % 4], x, y);
          vh[i] = x;
          vl[i] = y;
        }
        *gmem((bf16x8*)((bf16*)a.dzh + e0 + 8 * j)) = vh;
        *gmem((bf16x8*)((bf16*)a.dzl + e0 + 8 * j)) = vl;
      }
    }
  }
  if (part == 0 && gate) sG[t] = g;
  if (mean) {
    // dm rows over this thread's own region of sMt (no other thread reads it after the dots)
#pragma unroll
    for (int j = 0; j < PER / 4; ++j) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int cc = part * PER + 4 * j + i;
        sMt[t * LDM + cc] = am * gv[j][i] + ds * (float)qv8[j / 2][4 * (j % 2) + i];
      }
    }
  }
  if (mean || gate) {
    __syncthreads();
    if (mean && tid < NSEG * K) {
      float acc = 0.f;
#pragma unroll
      for (int r = 0; r < RPS; ++r) acc += sMt[(seg * RPS + r) * LDM + col];  // rows >= L are 0
      sD[seg][col] = acc;
    }
    if (gate) {
      // dlogit_t q_t rows over this thread's region of sMt (0 past the chunk), then column sums
      if (mean) __syncthreads();
#pragma unroll
      for (int j = 0; j < PER / 8; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) sMt[t * LDM + part * PER + 8 * j + i] = g * (float)qv8[j][i];
      __syncthreads();
      if (tid < NSEG * K) {
        float acc = 0.f;
#pragma unroll
        for (int r = 0; r < RPS; ++r) acc += sMt[(seg * RPS + r) * LDM + col];
        sW[seg][col] = acc;
      }
    }
    __syncthreads();
    if (tid < K) {
      float accd = 0.f, accw = 0.f;
      for (int sg = 0; sg < NSEG; ++sg) {
        accd += sD[sg][tid];
        accw += sW[sg][tid];
      }
      if (mean) a.dmsum[((long)gc * a.H + h) * K + tid] = accd;
      if (gate) dwp[tid] = accw;
    }
  }
  if (gate) {
    // db on the first whole wave without a dW column (wave 0 when K == 256)
    constexpr int DBW = K >= kThreads ? 0 : ((K + 63) / 64) * 64;
    if (tid >= DBW && tid < DBW + 64) {
      float v = 0.f;
      for (int t2 = tid - DBW; t2 < CB; t2 += 64) v += sG[t2];
      v = group_sum(v, 64);
      if (tid == DBW) a.db_part[(long)gc * a.H + h] = v;
    }
  }
}

// ===========================================================================
// cw_dq: grid N*H*(K/32)*nseg; forward walk of C (from the segment's start state).  Same roles as cw_fwd (state waves load, output waves
// store); for K <= 128 the staged tiles are double-buffered (two barriers per chunk, the stage of the
// next chunk overlapping the output rows of this one), for K = 256 one buffer and three barriers:
//   stage    state waves: dZ (hi/lo), K, C[:, cols] (hi/lo), row scalars, key sums
//   phase 1  score blocks (dZ K^T)^T = K_J dZ_I^T, kept for s <= t
//   phase 2  output waves: dq rows, then the load of their dqc slice of the next chunk (issued after
//            the stores, so that waiting for it one chunk later finds the stores long done);
//            state waves: C update
// ===========================================================================
template <int K>
__global__ __launch_bounds__(kThreads) void cw_dq_kernel(const WalkArgs a) {
  using W = Walk<K>;
  constexpr int CB = W::CB, NB = W::NB, NSW = W::NSW, NRT = W::NRT, TPW = W::TPW, LDK = W::LDK, LDA = W::LDA;
  constexpr int NLT = NSW * 64, NBUF = K > 128 ? 1 : 2;
  __shared__ __attribute__((aligned(16))) bf16 sZh_[NBUF][CB * LDK];  // dz rows, hi
  __shared__ __attribute__((aligned(16))) bf16 sZl_[NBUF][CB * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sK_[NBUF][CB * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sCh_[NBUF][32 * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sCl_[NBUF][32 * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sAh[CB * LDA];  // dz_t . k_s (s <= t), hi
  __shared__ __attribute__((aligned(16))) bf16 sAl[CB * LDA];
  __shared__ __attribute__((aligned(16))) f32x4 sR_[NBUF][CB];  // row scalars
  __shared__ float sMp_[NBUF][32], sWc[32];

  const int tid = threadIdx.x, w = wave_id();
  const WalkUnit u = walk_unit<K>(a);
  const bool mean = a.subtract_mean != 0, gate = a.gate_w != nullptr;
  const int sw = w - NB, lt = tid - NB * 64;

  f32x16 C[TPW];
  load_slice<K>(C, a.h0 ? a.h0 + (long)u.unit * K * K : nullptr, sw, u.c0, false);
  if (u.seg > 0) add_seg_slice<K>(C, a.segD, u.unit, u.nseg, 0, u.seg, sw, u.c0, false);
  if (tid < 32) sWc[tid] = gate ? a.gate_w[(long)u.h * K + u.c0 + tid] : 0.f;

  PrefetchDzRows<K, CB, NLT> pz;
  PrefetchRows<K, CB, NLT> pk;
  f32x4 prow;
  float pmp = 0.f;
  float gcol[16];  // output waves: dqc at this lane's (row, column) positions of the current chunk
  const int orow = 32 * w + acc_row(0);  // output waves: first row of this lane in a chunk
  auto issue_cols = [&](int c) {
    const long base = u.hb + (long)c * CB * u.rs + u.c0 + acc_col();
    load16(a.dqc32, (const bf16*)a.dqc16, base, u.rs, gcol, orow, min(CB, u.len - c * CB));
  };
  if (w < NB && u.cb < u.ce) issue_cols(u.cb);
  auto issue = [&](int c) {
    const int L = min(CB, u.len - c * CB);
    const long off = u.hb + (long)c * CB * u.rs;
    const long ti0 = (u.bos + (long)c * CB) * a.H + u.h;
    pz.load(a.dqc32 ? a.dqc32 + off : nullptr, a.dqc32 ? nullptr : (const bf16*)a.dqc16 + off, u.rs,
            a.sc + ti0 * 4, (long)a.H * 4, L, lt);
    pk.load((const bf16*)a.k + off, u.rs, L, lt);
    if (lt < CB) prow = *(const f32x4*)(a.sc + (ti0 + (long)min(lt, L - 1) * a.H) * 4);
    if (mean && lt >= 64 && lt < 96) pmp = a.mpre[((long)(u.gc0 + c) * a.H + u.h) * K + u.c0 + lt - 64];
  };
  if (sw >= 0 && u.cb < u.ce) issue(u.cb);

  for (int c = u.cb; c < u.ce; ++c) {
    const int t0 = c * CB, L = min(CB, u.len - t0), b = (NBUF == 2) ? (c & 1) : 0;
    bf16* sZh = sZh_[b];
    bf16* sZl = sZl_[b];
    bf16* sK = sK_[b];
    bf16* sCh = sCh_[b];
    bf16* sCl = sCl_[b];
    f32x4* sR = sR_[b];
    float* sMp = sMp_[b];
    if (sw >= 0) {
      pz.store(sZh, sZl, LDK, L, lt);
      pk.store(sK, LDK, L, lt);
      if (lt < CB) sR[lt] = (lt < L) ? prow : f32x4{};
      if (lt >= 64 && lt < 96) sMp[lt - 64] = pmp;
#pragma unroll
      for (int j = 0; j < TPW; ++j) {
        const int rt = sw + NSW * j;
        if (rt < NRT) acc_to_lds_t(C[j], sCh, sCl, LDK, rt * 32);
      }
    }
    __syncthreads();

    // ---- phase 1
    if (sw >= 0 && c + 1 < u.ce) issue(c + 1);
    if (w < W::NBLK) {
      const int I = blk_row(w), J = blk_col(w);
      f32x16 ah = zero16();
      const bf16* Kr = sK + J * 32 * LDK;
#pragma unroll 4
      for (int k0 = 0; k0 < K; k0 += 16) {
        const bf16x8 kf = frag_rm(Kr + k0, LDK);
        ah = mfma(kf, frag_rm(sZh + I * 32 * LDK + k0, LDK), ah);
        ah = mfma(kf, frag_rm(sZl + I * 32 * LDK + k0, LDK), ah);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (32 * J + acc_row(i) > 32 * I + acc_col()) ah[i] = 0.f;
      acc_to_lds_t(ah, sAh + I * 32 * LDA, sAl + I * 32 * LDA, LDA, 32 * J);
    }
    __syncthreads();

    // ---- phase 2
    if (w < NB) {
      const int I = w;
      f32x16 x = zero16(), cum = zero16();
      const bf16* Zh = sZh + I * 32 * LDK;
      const bf16* Zl = sZl + I * 32 * LDK;
#pragma unroll 4
      for (int k0 = 0; k0 < K; k0 += 16) {
        const bf16x8 zh = frag_rm(Zh + k0, LDK);
        const bf16x8 ch = frag_rm(sCh + k0, LDK);
        x = mfma(zh, ch, x);
        x = mfma(zh, frag_rm(sCl + k0, LDK), x);
        x = mfma(frag_rm(Zl + k0, LDK), ch, x);
      }
      for (int s0 = 0; s0 < 32 * (I + 1); s0 += 16) {
        const bf16x8 kf = frag32_tr(sK + s0 * LDK + u.c0, LDK);
        x = mfma(frag_rm(sAh + I * 32 * LDA + s0, LDA), kf, x);
        x = mfma(frag_rm(sAl + I * 32 * LDA + s0, LDA), kf, x);
        if (mean) cum = mfma(frag_tril_ones(32 * I, s0), kf, cum);
      }
      const int cc = acc_col();
      const float mc = sMp[cc], wc = sWc[cc];
      const int r0 = 32 * I + acc_row(0);
      const long rowbase = u.hb + (long)(t0 + r0) * u.rs + u.c0 + cc;
      float dsv[16], dlv[16], d[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const f32x4 r = sR[r0 + acc_drow(i)];
        dsv[i] = r[1];
        dlv[i] = r[2];
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        d[i] = gcol[i] + x[i];
        if (mean) d[i] += dsv[i] * (mc + cum[i]);
        if (gate) d[i] += dlv[i] * wc;
      }
      store16(a.dq32, (bf16*)a.dq, rowbase, u.rs, d, r0, L);
      if (c + 1 < u.ce) issue_cols(c + 1);
    } else {
      bf16x8 kc[CB / 16];
#pragma unroll
      for (int s = 0; s < CB / 16; ++s) kc[s] = frag32_tr(sK + s * 16 * LDK + u.c0, LDK);
#pragma unroll
      for (int j = 0; j < TPW; ++j) {
        const int rt = sw + NSW * j;
        if (rt < NRT) {
#pragma unroll
          for (int s = 0; s < CB / 16; ++s) C[j] = mfma(frag32_tr(sK + s * 16 * LDK + rt * 32, LDK), kc[s], C[j]);
        }
      }
    }
    if (NBUF == 1) __syncthreads();
  }
}

// ===========================================================================
// cw_dk: grid N*H*(K/32)*nseg; reverse walk of E = G + G^T (G = dC_T + sum of q dz^T over later
// chunks; the later segments enter through their totals, segG and segDM).
// The in-chunk suffix sums of dm_t = ds_t q_t - (s_t/pos_t) dz_t ride along the score products:
//   dk_j = K E + sum_{t>=j} (B1[j][t] + ds_t) q_t + sum_{t>=j} (B2[j][t] - s_t/pos_t) dz_t + carry,
// where the masked diagonal terms enter as their own hi/lo fragments (|s/pos| can exceed |q . k| by
// orders of magnitude, so they are not added into the score blocks before the split), and
// carry = dm_T + the per-chunk column sums of dm of the later chunks (from cw_rows).
// Roles as cw_dq:
//   stage    state waves: Q, K, dZ (hi/lo), E[:, cols] (hi/lo), row scalars, carry update
//   phase 1  score blocks B1 = dz_t . k_j, B2 = q_t . k_j (t >= j) as [j][t]
//   phase 2  output waves: dk rows, then the load of their dk_extra slice of the next chunk;
//            state waves: E += Q^T dZ[:, cols] + dZ^T Q[:, cols] (and G += Q^T dZ[:, cols] when
//            DH0: dC_0 is requested)
// ===========================================================================
template <int K, bool DH0>
__global__ __launch_bounds__(kThreads) void cw_dk_kernel(const WalkArgs a) {
  using W = Walk<K>;
  constexpr int CB = W::CB, NB = W::NB, NSW = W::NSW, NRT = W::NRT, TPW = W::TPW, LDK = W::LDK, LDA = W::LDA;
  constexpr int NLT = NSW * 64;
  __shared__ __attribute__((aligned(16))) bf16 sQ[CB * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sK[CB * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sZh[CB * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sZl[CB * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sEh[32 * LDK];  // E[:, cols] as [col][row]
  __shared__ __attribute__((aligned(16))) bf16 sEl[32 * LDK];
  __shared__ __attribute__((aligned(16))) bf16 sB1h[CB * LDA];  // [j][t] = dz_t . k_j (t >= j)
  __shared__ __attribute__((aligned(16))) bf16 sB1l[CB * LDA];
  __shared__ __attribute__((aligned(16))) bf16 sB2h[CB * LDA];  // [j][t] = q_t . k_j (t >= j)
  __shared__ __attribute__((aligned(16))) bf16 sB2l[CB * LDA];
  __shared__ __attribute__((aligned(16))) f32x4 sR[CB];
  __shared__ __attribute__((aligned(16))) float sDs[CB], sSp[CB];  // ds_t, -s_t/pos_t
  __shared__ float sCar[2][32];  // sum of dm over later chunks (+ dm_T), by chunk parity

  const int tid = threadIdx.x, w = wave_id(), l = lane_id();
  const WalkUnit u = walk_unit<K>(a);
  const bool mean = a.subtract_mean != 0;
  const int sw = w - NB, lt = tid - NB * 64;

  // E at the end of the segment: dC_T + dC_T^T (+ the later segments' G + G^T); G (dC_0, written
  // by the first segment) starts from dC_T + the later segments' G
  const bool first = u.seg == 0;
  f32x16 E[TPW], G[TPW];  // G is dead unless DH0
  {
    const float* dhf = a.dh_fin ? a.dh_fin + (long)u.unit * K * K : nullptr;
    f32x16 Tt[TPW];
    load_slice<K>(E, dhf, sw, u.c0, false);
    load_slice<K>(Tt, dhf, sw, u.c0, true);
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      if constexpr (DH0) G[j] = E[j];
      E[j] += Tt[j];
    }
    if (u.seg + 1 < u.nseg) {
      add_seg_slice<K>(E, a.segG, u.unit, u.nseg, u.seg + 1, u.nseg, sw, u.c0, true);
      if constexpr (DH0) add_seg_slice<K>(G, a.segG, u.unit, u.nseg, u.seg + 1, u.nseg, sw, u.c0, false);
    }
  }
  // carry lanes: loader threads lt in [64, 96) own column lt - 64 of the carry (dm_T + the later
  // segments' dm sums)
  const bool carl = lt >= 64 && lt < 96;
  if (carl) {
    float car = (mean && a.dm_fin) ? a.dm_fin[(long)u.unit * K + u.c0 + lt - 64] : 0.f;
    if (mean)
      for (int s2 = u.seg + 1; s2 < u.nseg; ++s2) car += a.segDM[((long)u.unit * u.nseg + s2) * K + u.c0 + lt - 64];
    sCar[0][lt - 64] = car;
  }

  PrefetchRows<K, CB, NLT> pq, pk;
  PrefetchDzRows<K, CB, NLT> pz;
  f32x4 prow;
  float pdm = 0.f;
  auto issue = [&](int c) {
    const int L = min(CB, u.len - c * CB);
    const long off = u.hb + (long)c * CB * u.rs;
    const long ti0 = (u.bos + (long)c * CB) * a.H + u.h;
    pq.load((const bf16*)a.q + off, u.rs, L, lt);
    pk.load((const bf16*)a.k + off, u.rs, L, lt);
    pz.load(a.dqc32 ? a.dqc32 + off : nullptr, a.dqc32 ? nullptr : (const bf16*)a.dqc16 + off, u.rs,
            a.sc + ti0 * 4, (long)a.H * 4, L, lt);
    if (lt < CB) prow = *(const f32x4*)(a.sc + (ti0 + (long)min(lt, L - 1) * a.H) * 4);
    if (mean && carl) pdm = a.dmsum[((long)(u.gc0 + c) * a.H + u.h) * K + u.c0 + lt - 64];
  };
  float xcol[16];  // output waves: dk_extra at this lane's (row, column) positions of the current chunk
  const int orow = 32 * w + acc_row(0);
  auto issue_cols = [&](int c) {
    const long base = u.hb + (long)c * CB * u.rs + u.c0 + acc_col();
    load16(a.dk_extra, nullptr, base, u.rs, xcol, orow, min(CB, u.len - c * CB));
  };
  if (u.cb < u.ce) {
    if (sw >= 0) issue(u.ce - 1);
    else if (a.dk_extra) issue_cols(u.ce - 1);
  }

  int p = 0;
  for (int c = u.ce - 1; c >= u.cb; --c, p ^= 1) {
    const int t0 = c * CB, L = min(CB, u.len - t0);
    if (sw >= 0) {
      pq.store(sQ, LDK, L, lt);
      pk.store(sK, LDK, L, lt);
      pz.store(sZh, sZl, LDK, L, lt);
      if (lt < CB) {
        const f32x4 r = (lt < L) ? prow : f32x4{};
        sR[lt] = r;
        sDs[lt] = r[1];
        sSp[lt] = r[3];
      }
      if (carl) sCar[p ^ 1][lt - 64] = sCar[p][lt - 64] + pdm;
#pragma unroll
      for (int j = 0; j < TPW; ++j) {
        const int rt = sw + NSW * j;
        if (rt < NRT) acc_to_lds_t(E[j], sEh, sEl, LDK, rt * 32);
      }
    }
    __syncthreads();

    // ---- phase 1
    if (sw >= 0 && c > u.cb) issue(c - 1);
    if (w < W::NBLK) {
      const int T = blk_row(w), J = blk_col(w);
      f32x16 b1h = zero16(), b2 = zero16();
      const bf16* Kr = sK + J * 32 * LDK;
#pragma unroll 4
      for (int k0 = 0; k0 < K; k0 += 16) {
        const bf16x8 kf = frag_rm(Kr + k0, LDK);
        b1h = mfma(frag_rm(sZh + T * 32 * LDK + k0, LDK), kf, b1h);
        b1h = mfma(frag_rm(sZl + T * 32 * LDK + k0, LDK), kf, b1h);
        b2 = mfma(frag_rm(sQ + T * 32 * LDK + k0, LDK), kf, b2);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (32 * T + acc_row(i) < 32 * J + acc_col()) {
          b1h[i] = 0.f;
          b2[i] = 0.f;
        }
      }
      acc_to_lds_t(b1h, sB1h + J * 32 * LDA, sB1l + J * 32 * LDA, LDA, 32 * T);
      acc_to_lds_t(b2, sB2h + J * 32 * LDA, sB2l + J * 32 * LDA, LDA, 32 * T);
    }
    __syncthreads();

    // ---- phase 2
    if (w < NB) {
      const int J = w;
      f32x16 x = zero16();
      const bf16* Kr = sK + J * 32 * LDK;
#pragma unroll 4
      for (int k0 = 0; k0 < K; k0 += 16) {
        const bf16x8 kf = frag_rm(Kr + k0, LDK);
        x = mfma(kf, frag_rm(sEh + k0, LDK), x);
        x = mfma(kf, frag_rm(sEl + k0, LDK), x);
      }
#pragma unroll 2
      for (int s0 = 32 * J; s0 < CB; s0 += 16) {
        const bf16x8 qf = frag32_tr(sQ + s0 * LDK + u.c0, LDK);
        x = mfma(frag_rm(sB1h + J * 32 * LDA + s0, LDA), qf, x);
        x = mfma(frag_rm(sB1l + J * 32 * LDA + s0, LDA), qf, x);
        const bf16x8 zhf = frag32_tr(sZh + s0 * LDK + u.c0, LDK);
        const bf16x8 b2h = frag_rm(sB2h + J * 32 * LDA + s0, LDA);
        x = mfma(b2h, zhf, x);
        const bf16x8 zlf = frag32_tr(sZl + s0 * LDK + u.c0, LDK);
        x = mfma(b2h, zlf, x);
        x = mfma(frag_rm(sB2l + J * 32 * LDA + s0, LDA), zhf, x);
        if (mean) {
          // masked diagonals: (j, t) -> ds_t [t >= j] against q, -s_t/pos_t [t >= j] against dz
          const int tb = s0 + ((l >> 5) << 3), jr = 32 * J + (l & 31);
          const f32x4 d0 = *(const f32x4*)(sDs + tb), d1 = *(const f32x4*)(sDs + tb + 4);
          const f32x4 p0 = *(const f32x4*)(sSp + tb), p1 = *(const f32x4*)(sSp + tb + 4);
          bf16x8 dh, dl, ph, pl;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const bool keep = tb + i >= jr;
            bf16 a1, a2, a3, a4;
            split2(keep ? (i < 4 ? d0[i] : d1[i - 4]) : 0.f, a1, a2);
            split2(keep ? (i < 4 ? p0[i] : p1[i - 4]) : 0.f, a3, a4);
            dh[i] = a1;
            dl[i] = a2;
            ph[i] = a3;
            pl[i] = a4;
          }
          x = mfma(dh, qf, x);
          x = mfma(dl, qf, x);
          x = mfma(ph, zhf, x);
          x = mfma(ph, zlf, x);
          x = mfma(pl, zhf, x);
        }
      }
      const float car = sCar[p][acc_col()];
      const int r0 = 32 * J + acc_row(0);
      const long rowbase = u.hb + (long)(t0 + r0) * u.rs + u.c0 + acc_col();
      float d[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) d[i] = x[i] + car + (a.dk_extra ? xcol[i] : 0.f);
      store16(a.dk32, (bf16*)a.dk, rowbase, u.rs, d, r0, L);
      if (a.dk_extra && c > u.cb) issue_cols(c - 1);
    } else {
#pragma unroll
      for (int s = 0; s < CB / 16; ++s) {
        const bf16x8 qc = frag32_tr(sQ + s * 16 * LDK + u.c0, LDK);
        const bf16x8 zc = frag32_tr(sZh + s * 16 * LDK + u.c0, LDK);
        const bf16x8 zcl = frag32_tr(sZl + s * 16 * LDK + u.c0, LDK);
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
          const int rt = sw + NSW * j;
          if (rt < NRT) {
            const bf16x8 qr = frag32_tr(sQ + s * 16 * LDK + rt * 32, LDK);   // (r, t) = q_t[rt*32 + r]
            const bf16x8 zr = frag32_tr(sZh + s * 16 * LDK + rt * 32, LDK);  // (r, t) = dz_t[rt*32 + r]
            const bf16x8 zrl = frag32_tr(sZl + s * 16 * LDK + rt * 32, LDK);
            if (DH0 && first) {
              G[j] = mfma(qr, zc, G[j]);
              G[j] = mfma(qr, zcl, G[j]);
            }
            E[j] = mfma(qr, zc, E[j]);
            E[j] = mfma(qr, zcl, E[j]);
            E[j] = mfma(zr, qc, E[j]);
            E[j] = mfma(zrl, qc, E[j]);
          }
        }
      }
    }
    __syncthreads();
  }

  if constexpr (DH0) {
    if (first) store_slice<K>(G, a.dh0 + (long)u.unit * K * K, sw, u.c0);
  }
  if (first && a.dm0 && carl) a.dm0[(long)u.unit * K + u.c0 + lt - 64] = mean ? sCar[p][lt - 64] : 0.f;
}

// ===========================================================================
// launcher
// ===========================================================================
namespace {

template <int K>
hipError_t cwalk_k(int stage, const WalkArgs& a, hipStream_t st) {
  const long units = (long)a.N * a.H * (K / 32) * (a.segD ? a.nseg : 1);
  switch (stage) {
    case kWalkFwd:
      if (units > 0) hipLaunchKernelGGL(cw_fwd_kernel<K>, dim3((unsigned)units), dim3(kThreads), 0, st, a);
      break;
    case kWalkRows:
      if ((long)a.NTG * a.H > 0)
        hipLaunchKernelGGL(cw_rows_kernel<K>, dim3((unsigned)((long)a.NTG * a.H)), dim3(kThreads), 0, st, a);
      break;
    case kWalkDq:
      if (units > 0) hipLaunchKernelGGL(cw_dq_kernel<K>, dim3((unsigned)units), dim3(kThreads), 0, st, a);
      break;
    case kWalkDk:
      if (units > 0) {
        if (a.dh0) hipLaunchKernelGGL((cw_dk_kernel<K, true>), dim3((unsigned)units), dim3(kThreads), 0, st, a);
        else hipLaunchKernelGGL((cw_dk_kernel<K, false>), dim3((unsigned)units), dim3(kThreads), 0, st, a);
      }
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_cwalk(int stage, const WalkArgs& a, hipStream_t st) {
  switch (a.K) {
    // (K = 64 and 128 run as segment walks)
    case 32: return cwalk_k<32>(stage, a, st);
    case 256: return cwalk_k<256>(stage, a, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ccq
