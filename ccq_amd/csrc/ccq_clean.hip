// CCQ read-side cleaning operator on gfx950: forward and backward sweeps.
//
// Mathematics (per sequence and head; reference ccq/ops/common/fused_read.py:11-25):
//   h_t = h_0 + sum_{j<=t} k_j k_j^T          m_t = m_0 + sum_{j<=t} k_j
//   z_t = h_t^T q_t     s_t = m_t . q_t      corr_t = z_t/pos_t - s_t m_t/pos_t^2
//   q_clean_t = q_t - lambda_t corr_t
//
// Work decomposition: one workgroup owns one (sequence, head, 32-column block of
// the K x K state) and walks the sequence in 32-token steps.  Its slice of the
// state lives in MFMA accumulators (fp32) for the whole walk; a hi/lo bf16 snapshot
// of it is kept in LDS as the MFMA operand of the next step (so z, and with it
// dlambda = -dqc . corr, keeps ~16 significant bits even when h0 dominates).
// The next step's q/k rows are prefetched into registers while a step computes.
//
// Per 32-token step (rows t, state columns c in the block):
//   A   = Q K^T (causal incl. diagonal)                 -> s_t = m_prev.q_t + rowsum(A)
//   Z   = Q H[:, c] + A K[:, c]                         (z_t restricted to the block)
//   cum = m_prev[c] + L1 K[:, c]       (L1 = 0/1 lower-triangular matrix: a prefix sum on MFMA)
//   H[:, c] += K^T K[:, c]
#include "ccq_tile.h"
#include "ccq_params.h"

namespace ccq {

namespace {

constexpr int kC = 32;   // tokens per sweep step
constexpr int kCB = 32;  // state columns per workgroup

// Carve a byte buffer into consecutive arrays (16-byte aligned).
struct Carver {
  char* p;
  template <typename T>
  __device__ __forceinline__ T* take(int n) {
    T* r = (T*)p;
    p += ((long)n * sizeof(T) + 15) & ~15L;
    return r;
  }
};

template <int K>
struct FwdLds {
  static constexpr int LDK = K + 8, LDC = kC + 8, LDF = kC + 1;
  static constexpr long bytes() {
    return 2L * (kC * LDK) * 2 + (long)K * LDC * 2 + 2L * kCB * LDK * 2 + 2L * kC * LDC * 2 +
           2L * kC * LDF * 4 + (long)K * 4 + 3L * kC * 4 + 16 * 14;
  }
};

}  // namespace

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
template <int K>
__global__ __launch_bounds__(kThreads) void ccq_clean_fwd_kernel(const CleanFwdArgs a) {
  constexpr int C = kC, CB = kCB, NCB = K / CB, NRT = K / 32, TPW = (NRT + 3) / 4;
  constexpr int LDK = FwdLds<K>::LDK, LDC = FwdLds<K>::LDC, LDF = FwdLds<K>::LDF;
  __shared__ __attribute__((aligned(16))) char smem[FwdLds<K>::bytes()];
  Carver cv{smem};
  bf16* sQ = cv.take<bf16>(C * LDK);
  bf16* sK = cv.take<bf16>(C * LDK);
  bf16* sKT = cv.take<bf16>(K * LDC);
  bf16* sHT = cv.take<bf16>(CB * LDK);   // H[:, block]^T, hi part
  bf16* sHTl = cv.take<bf16>(CB * LDK);  // lo part
  bf16* sA = cv.take<bf16>(C * LDC);
  bf16* sAl = cv.take<bf16>(C * LDC);
  float* sAf = cv.take<float>(C * LDF);
  float* sCum = cv.take<float>(C * LDF);
  float* sM = cv.take<float>(K);
  float* sLam = cv.take<float>(C);
  float* sPos = cv.take<float>(C);
  float* sS = cv.take<float>(C);

  const int tid = threadIdx.x, w = wave_id();
  int unit, cb;
  xcd_map(blockIdx.x, NCB, a.N * a.H, unit, cb);
  const int n = unit / a.H, h = unit % a.H;
  long bos;
  int len;
  seq_bounds(a.cu, n, a.T, bos, len);
  const long rs = (long)a.H * K;
  const long base = (bos * a.H + h) * (long)K;
  const int col0 = cb * CB;
  const bool mean = a.subtract_mean != 0;
  const bf16* qg = (const bf16*)a.q + base;
  const bf16* kg = (const bf16*)a.k + base;

  f32x16 Hs[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    Hs[j] = zero16();
    const int rt = w + 4 * j;
    if (rt < NRT && a.h0) {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        Hs[j][i] = a.h0[((long)unit * K + rt * 32 + acc_row(i)) * K + col0 + acc_col()];
    }
  }
  for (int kk = tid; kk < K; kk += kThreads) sM[kk] = (mean && a.m0) ? a.m0[(long)unit * K + kk] : 0.f;
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int rt = w + 4 * j;
    if (rt < NRT) {
#pragma unroll
      for (int i = 0; i < 16; ++i) split2(Hs[j][i], sHT[acc_col() * LDK + rt * 32 + acc_row(i)], sHTl[acc_col() * LDK + rt * 32 + acc_row(i)]);
    }
  }

  PrefetchBf16<K, C> pq, pk;
  pq.load(qg, rs, min(C, len));
  pk.load(kg, rs, min(C, len));

  for (int t0 = 0; t0 < len; t0 += C) {
    const int L = min(C, len - t0);
    pq.store(sQ, LDK, nullptr, 0);
    pk.store(sK, LDK, sKT, LDC);
    if (tid < C) {
      const float pos = (float)(t0 + tid + 1 + a.pos_off);
      sPos[tid] = pos < 1.f ? 1.f : pos;
      if (!a.gate_w) sLam[tid] = (tid < L) ? a.lam[(bos + t0 + tid) * a.H + h] : 0.f;
    }
    __syncthreads();
    if (t0 + C < len) {
      const int Ln = min(C, len - t0 - C);
      pq.load(qg + (long)(t0 + C) * rs, rs, Ln);
      pk.load(kg + (long)(t0 + C) * rs, rs, Ln);
    }
    if (a.gate_w) {
      const int r = tid >> 3, part = tid & 7;
      float d = 0.f;
      for (int kk = part; kk < K; kk += 8) d += (float)sQ[r * LDK + kk] * a.gate_w[(long)h * K + kk];
      d = group_sum(d, 8);
      if (part == 0) {
        const float lv = (r < L) ? sigmoidf_(d + a.gate_b[h]) : 0.f;
        sLam[r] = lv;
        if (a.lam_out && cb == 0 && r < L) a.lam_out[(bos + t0 + r) * a.H + h] = lv;
      }
    }

    f32x16 zacc = zero16();
    if (w == 0) {
      f32x16 acc = zero16();
      mma_rr(acc, sQ, LDK, sK, LDK, K);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = acc_row(i), c = acc_col();
        const float v = (c <= r) ? acc[i] : 0.f;
        sAf[r * LDF + c] = v;
        split2(v, sA[r * LDC + c], sAl[r * LDC + c]);
      }
    } else if (w == 1) {
      mma_rr(zacc, sQ, LDK, sHT, LDK, K);
      mma_rr(zacc, sQ, LDK, sHTl, LDK, K);
    } else if (w == 2 && mean) {
      f32x16 acc = zero16();
#pragma unroll
      for (int k0 = 0; k0 < C; k0 += 16) acc = mfma(frag_tril_ones(0, k0), frag_rm(sKT + col0 * LDC + k0, LDC), acc);
#pragma unroll
      for (int i = 0; i < 16; ++i) sCum[acc_row(i) * LDF + acc_col()] = acc[i];
    }
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int rt = w + 4 * j;
      if (rt < NRT) mma_rr(Hs[j], sKT + rt * 32 * LDC, LDC, sKT + col0 * LDC, LDC, C);
    }
    __syncthreads();

    if (mean) {
      const int r = tid >> 3, part = tid & 7;
      float s = 0.f;
      for (int kk = part; kk < K; kk += 8) s += sM[kk] * (float)sQ[r * LDK + kk];
      for (int j = part; j < C; j += 8) s += sAf[r * LDF + j];
      s = group_sum(s, 8);
      if (part == 0) sS[r] = s;
    }
    __syncthreads();

    if (w == 1) {
      mma_rr(zacc, sA, LDC, sKT + col0 * LDC, LDC, C);
      mma_rr(zacc, sAl, LDC, sKT + col0 * LDC, LDC, C);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = acc_row(i), c = acc_col();
        if (r < L) {
          const float p = sPos[r];
          float corr = zacc[i] / p;
          if (mean) corr -= sS[r] / (p * p) * (sM[col0 + c] + sCum[r * LDF + c]);
          const float out = (float)sQ[r * LDK + col0 + c] - sLam[r] * corr;
          const long gi = base + (long)(t0 + r) * rs + col0 + c;
          if (a.qc) ((bf16*)a.qc)[gi] = (bf16)out;
          if (a.qc32) a.qc32[gi] = out;
        }
      }
    }
    float mnew = 0.f;
    if (mean && tid < K) {
      float cs = 0.f;
      for (int r = 0; r < C; ++r) cs += (float)sK[r * LDK + tid];
      mnew = sM[tid] + cs;
    }
    __syncthreads();
    if (mean && tid < K) sM[tid] = mnew;
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int rt = w + 4 * j;
      if (rt < NRT) {
#pragma unroll
        for (int i = 0; i < 16; ++i) split2(Hs[j][i], sHT[acc_col() * LDK + rt * 32 + acc_row(i)], sHTl[acc_col() * LDK + rt * 32 + acc_row(i)]);
      }
    }
    __syncthreads();
  }

  if (a.h_fin) {
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int rt = w + 4 * j;
      if (rt < NRT) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
          a.h_fin[((long)unit * K + rt * 32 + acc_row(i)) * K + col0 + acc_col()] = Hs[j][i];
      }
    }
  }
  if (a.m_fin && mean && cb == 0) {
    for (int kk = tid; kk < K; kk += kThreads) a.m_fin[(long)unit * K + kk] = sM[kk];
  }
}

// ---------------------------------------------------------------------------
// backward
//
// Closed-form gradients (reference ccq/ops/common/fused_read.py:18-25), with
// dz_t = -lambda_t dqc_t/pos_t (= F_t dqc_t):
//   dlambda_t = -dqc_t . corr_t
//   ds_t = lambda_t (dqc_t.m_t)/pos_t^2 = -(m_prev.dz_t + rowsum(B)_t)/pos_t,   B = dZ K^T (causal)
//   dm_t = lambda_t s_t dqc_t/pos_t^2 + ds_t q_t
//   dq_t = dqc_t + ds_t m_t + h_t dz_t          = dqc + ds cum + dZ H_prev + B K
//   dk_j = sum_{t>=j} [q_t (k_j.dz_t) + dz_t (k_j.q_t) + dm_t]
//        = (A^T dZ + B^T Q + U1 dm)_j + K E_next + carry(dm)
// blockIdx.y == 0: forward walk (dq, partial dlambda).  blockIdx.y == 1: reverse walk
// carrying E = G + G^T with G = sum_{later} q dz^T + dh_final (dk, dh0, dm0).
// ---------------------------------------------------------------------------

namespace {

template <int K>
struct BwdLds {
  static constexpr int LDK = K + 8, LDC = kC + 8, LDF = kC + 1, LDG = K + 4, LDZ = kC + 1, LDE = K + 1;
  static constexpr long fwd_bytes() {
    return 2L * (kC * LDK) * 2 + (long)K * LDC * 2 + 2L * kCB * LDK * 2 + (long)kC * LDG * 4 +
           2L * kC * LDC * 2 + 4L * kC * LDF * 4 + (long)K * 4 + 8L * kC * 4 + 16 * 22;
  }
  static constexpr long rev_bytes() {
    return 2L * K * LDC * 2 + (long)kC * LDK * 2 + (long)K * LDZ * 4 + (long)kCB * LDE * 4 + 2L * kC * LDC * 2 +
           3L * kC * LDF * 4 + 2L * K * 4 + (long)kCB * 4 + 8L * kC * 4 + 16 * 22;
  }
  static constexpr long bytes() { return fwd_bytes() > rev_bytes() ? fwd_bytes() : rev_bytes(); }
};

// fp32 operand with a per-row scale (row = lane's row r0 + l%32), element (r, k) at p[r * ld + k].
__device__ __forceinline__ void frag_rm_f32_rs(const float* p, int ld, float rscale, bf16x8& hi, bf16x8& lo) {
  const int l = lane_id();
  const float* q = p + (l & 31) * ld + ((l >> 5) << 3);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    bf16 hh, oo;
    split2(q[i] * rscale, hh, oo);
    hi[i] = hh;
    lo[i] = oo;
  }
}

// fp32 operand stored transposed, element (r, k) at p[k * ld + r], scaled by rs[r] (row scale).
__device__ __forceinline__ void frag_cm_f32_rs(const float* p, int ld, const float* rsc, bf16x8& hi, bf16x8& lo) {
  const int l = lane_id();
  const float s = rsc[l & 31];
  const float* q = p + ((l >> 5) << 3) * ld + (l & 31);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    bf16 hh, oo;
    split2(q[i * ld] * s, hh, oo);
    hi[i] = hh;
    lo[i] = oo;
  }
}

}  // namespace

template <int K>
__global__ __launch_bounds__(kThreads) void ccq_clean_bwd_kernel(const CleanBwdArgs a) {
  constexpr int C = kC, CB = kCB, NCB = K / CB, NRT = K / 32, TPW = (NRT + 3) / 4;
  using LD = BwdLds<K>;
  constexpr int LDK = LD::LDK, LDC = LD::LDC, LDF = LD::LDF, LDG = LD::LDG, LDZ = LD::LDZ, LDE = LD::LDE;
  __shared__ __attribute__((aligned(16))) char smem[LD::bytes()];

  const int tid = threadIdx.x, w = wave_id();
  int unit, cb;
  xcd_map(blockIdx.x, NCB, a.N * a.H, unit, cb);
  const int n = unit / a.H, h = unit % a.H;
  long bos;
  int len;
  seq_bounds(a.cu, n, a.T, bos, len);
  const long rs = (long)a.H * K;
  const long base = (bos * a.H + h) * (long)K;
  const int col0 = cb * CB;
  const bool mean = a.subtract_mean != 0;
  const bf16* qg = (const bf16*)a.q + base;
  const bf16* kg = (const bf16*)a.k + base;
  const float* g32 = a.dqc32 ? a.dqc32 + base : nullptr;
  const bf16* g16 = a.dqc16 ? (const bf16*)a.dqc16 + base : nullptr;
  const bool is32 = g32 != nullptr;

  if (blockIdx.y == 0) {
    // ======================= forward walk: dq, dlambda =======================
    Carver cv{smem};
    bf16* sQ = cv.take<bf16>(C * LDK);
    bf16* sK = cv.take<bf16>(C * LDK);
    bf16* sKT = cv.take<bf16>(K * LDC);
    bf16* sHT = cv.take<bf16>(CB * LDK);
    bf16* sHTl = cv.take<bf16>(CB * LDK);
    float* sG = cv.take<float>(C * LDG);
    bf16* sA = cv.take<bf16>(C * LDC);
    bf16* sAl = cv.take<bf16>(C * LDC);
    float* sAf = cv.take<float>(C * LDF);
    float* sBf = cv.take<float>(C * LDF);
    float* sCum = cv.take<float>(C * LDF);
    float* sRed = cv.take<float>(C * LDF);
    float* sM = cv.take<float>(K);
    float* sLam = cv.take<float>(C);
    float* sPos = cv.take<float>(C);
    float* sF = cv.take<float>(C);
    float* sS = cv.take<float>(C);
    float* sDS = cv.take<float>(C);

    f32x16 Hs[TPW];
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      Hs[j] = zero16();
      const int rt = w + 4 * j;
      if (rt < NRT && a.h0) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
          Hs[j][i] = a.h0[((long)unit * K + rt * 32 + acc_row(i)) * K + col0 + acc_col()];
      }
    }
    for (int kk = tid; kk < K; kk += kThreads) sM[kk] = (mean && a.m0) ? a.m0[(long)unit * K + kk] : 0.f;
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int rt = w + 4 * j;
      if (rt < NRT) {
#pragma unroll
        for (int i = 0; i < 16; ++i) split2(Hs[j][i], sHT[acc_col() * LDK + rt * 32 + acc_row(i)], sHTl[acc_col() * LDK + rt * 32 + acc_row(i)]);
      }
    }

    PrefetchBf16<K, C> pq, pk;
    PrefetchGrad<K, C> pg;
    pq.load(qg, rs, min(C, len));
    pk.load(kg, rs, min(C, len));
    pg.load(g32, g16, rs, min(C, len));

    for (int t0 = 0; t0 < len; t0 += C) {
      const int L = min(C, len - t0);
      pq.store(sQ, LDK, nullptr, 0);
      pk.store(sK, LDK, sKT, LDC);
      pg.store(is32, sG, LDG);
      if (tid < C) {
        float pos = (float)(t0 + tid + 1 + a.pos_off);
        pos = pos < 1.f ? 1.f : pos;
        const float lm = (tid < L) ? a.lam[(bos + t0 + tid) * a.H + h] : 0.f;
        sPos[tid] = pos;
        sLam[tid] = lm;
        sF[tid] = -lm / pos;
      }
      __syncthreads();
      if (t0 + C < len) {
        const int Ln = min(C, len - t0 - C);
        pq.load(qg + (long)(t0 + C) * rs, rs, Ln);
        pk.load(kg + (long)(t0 + C) * rs, rs, Ln);
        pg.load(g32 ? g32 + (long)(t0 + C) * rs : nullptr, g16 ? g16 + (long)(t0 + C) * rs : nullptr, rs, Ln);
      }

      f32x16 zacc = zero16(), yacc = zero16();
      if (w == 0) {
        f32x16 acc = zero16();
        mma_rr(acc, sQ, LDK, sK, LDK, K);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int r = acc_row(i), c = acc_col();
          const float v = (c <= r) ? acc[i] : 0.f;
          sAf[r * LDF + c] = v;
          split2(v, sA[r * LDC + c], sAl[r * LDC + c]);
        }
        if (mean) {
          f32x16 cacc = zero16();
#pragma unroll
          for (int k0 = 0; k0 < C; k0 += 16)
            cacc = mfma(frag_tril_ones(0, k0), frag_rm(sKT + col0 * LDC + k0, LDC), cacc);
#pragma unroll
          for (int i = 0; i < 16; ++i) sCum[acc_row(i) * LDF + acc_col()] = cacc[i];
        }
      } else if (w == 1) {
        // B = dZ K^T (causal), dZ rows = F_r * dqc_r (hi/lo)
        f32x16 acc = zero16();
        const float fr = sF[lane_id() & 31];
        for (int k0 = 0; k0 < K; k0 += 16) {
          bf16x8 hi, lo;
          frag_rm_f32_rs(sG + k0, LDG, fr, hi, lo);
          const bf16x8 b = frag_rm(sK + k0, LDK);
          acc = mfma(hi, b, acc);
          acc = mfma(lo, b, acc);
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int r = acc_row(i), c = acc_col();
          sBf[r * LDF + c] = (c <= r) ? acc[i] : 0.f;
        }
      } else if (w == 2) {
        mma_rr(zacc, sQ, LDK, sHT, LDK, K);
        mma_rr(zacc, sQ, LDK, sHTl, LDK, K);
      } else {
        // dqc H_prev (hi/lo); the row scale F is applied afterwards
        for (int k0 = 0; k0 < K; k0 += 16) {
          bf16x8 hi, lo;
          frag_rm_f32(sG + k0, LDG, hi, lo);
          const bf16x8 b = frag_rm(sHT + k0, LDK);
          yacc = mfma(hi, b, yacc);
          yacc = mfma(lo, b, yacc);
          yacc = mfma(hi, frag_rm(sHTl + k0, LDK), yacc);
        }
      }
#pragma unroll
      for (int j = 0; j < TPW; ++j) {
        const int rt = w + 4 * j;
        if (rt < NRT) mma_rr(Hs[j], sKT + rt * 32 * LDC, LDC, sKT + col0 * LDC, LDC, C);
      }
      __syncthreads();

      {
        // s = m_prev.q + rowsum(A);  ds = -(F (m_prev.dqc) + rowsum(B)) / pos  (no division by F)
        const int r = tid >> 3, part = tid & 7;
        float s = 0.f, rbB = 0.f, mg = 0.f;
        if (mean) {
          for (int kk = part; kk < K; kk += 8) {
            s += sM[kk] * (float)sQ[r * LDK + kk];
            mg += sM[kk] * sG[r * LDG + kk];
          }
          for (int j = part; j < C; j += 8) {
            s += sAf[r * LDF + j];
            rbB += sBf[r * LDF + j];
          }
        }
        s = group_sum(s, 8);
        rbB = group_sum(rbB, 8);
        mg = group_sum(mg, 8);
        if (part == 0) {
          sS[r] = s;
          sDS[r] = mean ? -(sF[r] * mg + rbB) / sPos[r] : 0.f;
        }
      }
      __syncthreads();

      if (w == 2) {
        mma_rr(zacc, sA, LDC, sKT + col0 * LDC, LDC, C);
        mma_rr(zacc, sAl, LDC, sKT + col0 * LDC, LDC, C);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int r = acc_row(i), c = acc_col();
          const float p = sPos[r];
          float corr = zacc[i] / p;
          if (mean) corr -= sS[r] / (p * p) * (sM[col0 + c] + sCum[r * LDF + c]);
          sRed[r * LDF + c] = sG[r * LDG + col0 + c] * corr;
        }
      } else if (w == 3) {
#pragma unroll
        for (int i = 0; i < 16; ++i) yacc[i] *= sF[acc_row(i)];
        for (int k0 = 0; k0 < C; k0 += 16) {
          bf16x8 hi, lo;
          frag_rm_f32(sBf + k0, LDF, hi, lo);
          const bf16x8 b = frag_rm(sKT + col0 * LDC + k0, LDC);
          yacc = mfma(hi, b, yacc);
          yacc = mfma(lo, b, yacc);
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int r = acc_row(i), c = acc_col();
          if (r < L) {
            float d = sG[r * LDG + col0 + c] + yacc[i];
            if (mean) d += sDS[r] * (sM[col0 + c] + sCum[r * LDF + c]);
            const long gi = base + (long)(t0 + r) * rs + col0 + c;
            if (a.dq) ((bf16*)a.dq)[gi] = (bf16)d;
            if (a.dq32) a.dq32[gi] = d;
          }
        }
      }
      float mnew = 0.f;
      if (mean && tid < K) {
        float cs = 0.f;
        for (int r = 0; r < C; ++r) cs += (float)sK[r * LDK + tid];
        mnew = sM[tid] + cs;
      }
      __syncthreads();
      if (tid < C && tid < L) {
        float s = 0.f;
        for (int c = 0; c < CB; ++c) s += sRed[tid * LDF + c];
        a.dlam_part[(long)cb * a.ntok * a.H + (bos + t0 + tid) * a.H + h] = -s;
      }
      if (mean && tid < K) sM[tid] = mnew;
#pragma unroll
      for (int j = 0; j < TPW; ++j) {
        const int rt = w + 4 * j;
        if (rt < NRT) {
#pragma unroll
          for (int i = 0; i < 16; ++i) split2(Hs[j][i], sHT[acc_col() * LDK + rt * 32 + acc_row(i)], sHTl[acc_col() * LDK + rt * 32 + acc_row(i)]);
        }
      }
      __syncthreads();
    }
    return;
  }

  // ======================= reverse walk: dk, dh0, dm0 =======================
  Carver cv{smem};
  bf16* sQT = cv.take<bf16>(K * LDC);
  bf16* sKT = cv.take<bf16>(K * LDC);
  bf16* sK = cv.take<bf16>(C * LDK);
  float* sGT = cv.take<float>(K * LDZ);   // dqc stored transposed [k][t]
  float* sET = cv.take<float>(CB * LDE);  // E[:, block] stored [c][k]
  bf16* sA = cv.take<bf16>(C * LDC);
  bf16* sAl = cv.take<bf16>(C * LDC);
  float* sAf = cv.take<float>(C * LDF);
  float* sBf = cv.take<float>(C * LDF);
  float* sDMT = cv.take<float>(CB * LDF);  // dm[:, block] stored [c][t]
  float* sMc = cv.take<float>(K);          // key sum after this step
  float* sMp = cv.take<float>(K);          // key sum before this step
  float* sDmc = cv.take<float>(CB);        // sum of dm over later steps (+ dm_final)
  float* sLam = cv.take<float>(C);
  float* sPos = cv.take<float>(C);
  float* sF = cv.take<float>(C);
  float* sS = cv.take<float>(C);
  float* sDS = cv.take<float>(C);
  float* sDMG = cv.take<float>(C);

  f32x16 Gs[TPW], Gt[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    Gs[j] = zero16();
    Gt[j] = zero16();
    const int rt = w + 4 * j;
    if (rt < NRT && a.dh_fin) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = rt * 32 + acc_row(i), c = col0 + acc_col();
        Gs[j][i] = a.dh_fin[((long)unit * K + row) * K + c];
        Gt[j][i] = a.dh_fin[((long)unit * K + c) * K + row];
      }
    }
  }
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int rt = w + 4 * j;
    if (rt < NRT) {
#pragma unroll
      for (int i = 0; i < 16; ++i) sET[acc_col() * LDE + rt * 32 + acc_row(i)] = Gs[j][i] + Gt[j][i];
    }
  }
  for (int kk = tid; kk < K; kk += kThreads) sMc[kk] = (mean && a.m_end) ? a.m_end[(long)unit * K + kk] : 0.f;
  if (tid < CB) sDmc[tid] = (mean && a.dm_fin) ? a.dm_fin[(long)unit * K + col0 + tid] : 0.f;

  const int last = len > 0 ? ((len - 1) / C) * C : -C;
  PrefetchBf16<K, C> pq, pk;
  PrefetchGrad<K, C> pg;
  if (last >= 0) {
    const int L0 = len - last;
    pq.load(qg + (long)last * rs, rs, L0);
    pk.load(kg + (long)last * rs, rs, L0);
    pg.load(g32 ? g32 + (long)last * rs : nullptr, g16 ? g16 + (long)last * rs : nullptr, rs, L0);
  }

  for (int t0 = last; t0 >= 0; t0 -= C) {
    const int L = min(C, len - t0);
    pq.store(nullptr, 0, sQT, LDC);
    pk.store(sK, LDK, sKT, LDC);
    // dqc transposed into fp32 LDS
    if (is32) {
      pg.f.store(nullptr, 0, sGT, LDZ);
    } else {
#pragma unroll
      for (int j = 0; j < PrefetchBf16<K, C>::N; ++j) {
        const int idx = threadIdx.x + j * kThreads;
        if (idx >= C * (K / 8)) continue;
        const int r = idx / (K / 8), c = (idx % (K / 8)) * 8;
#pragma unroll
        for (int i = 0; i < 8; ++i) sGT[(c + i) * LDZ + r] = (float)pg.b.v[j][i];
      }
    }
    if (tid < C) {
      float pos = (float)(t0 + tid + 1 + a.pos_off);
      pos = pos < 1.f ? 1.f : pos;
      const float lm = (tid < L) ? a.lam[(bos + t0 + tid) * a.H + h] : 0.f;
      sPos[tid] = pos;
      sLam[tid] = lm;
      sF[tid] = -lm / pos;
    }
    __syncthreads();
    if (t0 - C >= 0) {
      const int tn = t0 - C;
      pq.load(qg + (long)tn * rs, rs, C);
      pk.load(kg + (long)tn * rs, rs, C);
      pg.load(g32 ? g32 + (long)tn * rs : nullptr, g16 ? g16 + (long)tn * rs : nullptr, rs, C);
    }
    if (mean && tid < K) {
      float cs = 0.f;
      for (int r = 0; r < C; ++r) cs += (float)sK[r * LDK + tid];
      sMp[tid] = sMc[tid] - cs;
    }
    if (w == 0) {
      f32x16 acc = zero16();
      mma_cr(acc, sQT, LDC, sK, LDK, K);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = acc_row(i), c = acc_col();
        const float v = (c <= r) ? acc[i] : 0.f;
        sAf[r * LDF + c] = v;
        split2(v, sA[r * LDC + c], sAl[r * LDC + c]);
      }
    } else if (w == 1) {
      f32x16 acc = zero16();
      for (int k0 = 0; k0 < K; k0 += 16) {
        bf16x8 hi, lo;
        frag_cm_f32_rs(sGT + k0 * LDZ, LDZ, sF, hi, lo);
        const bf16x8 b = frag_rm(sK + k0, LDK);
        acc = mfma(hi, b, acc);
        acc = mfma(lo, b, acc);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = acc_row(i), c = acc_col();
        sBf[r * LDF + c] = (c <= r) ? acc[i] : 0.f;
      }
    }
    __syncthreads();

    if (mean) {
      const int r = tid >> 3, part = tid & 7;
      float s = 0.f, rbB = 0.f, mg = 0.f;
      for (int kk = part; kk < K; kk += 8) {
        s += sMp[kk] * (float)sQT[kk * LDC + r];
        mg += sMp[kk] * sGT[kk * LDZ + r];
      }
      for (int j = part; j < C; j += 8) {
        s += sAf[r * LDF + j];
        rbB += sBf[r * LDF + j];
      }
      s = group_sum(s, 8);
      rbB = group_sum(rbB, 8);
      mg = group_sum(mg, 8);
      if (part == 0) {
        const float p = sPos[r];
        sS[r] = s;
        sDS[r] = -(sF[r] * mg + rbB) / p;
        sDMG[r] = sLam[r] * s / (p * p);
      }
    }
    __syncthreads();
    if (mean) {
      for (int idx = tid; idx < C * CB; idx += kThreads) {
        const int r = idx / CB, c = idx % CB;
        sDMT[c * LDF + r] = sDMG[r] * sGT[(col0 + c) * LDZ + r] + sDS[r] * (float)sQT[(col0 + c) * LDC + r];
      }
    } else {
      for (int idx = tid; idx < C * CB; idx += kThreads) sDMT[(idx % CB) * LDF + idx / CB] = 0.f;
    }
    __syncthreads();

    if (w == 0) {
      f32x16 acc = zero16();
      // A^T dZ[:, block]
      for (int k0 = 0; k0 < C; k0 += 16) {
        const bf16x8 av = frag_cm(sA + k0 * LDC, LDC);
        bf16x8 hi, lo;
        frag_rm_f32_ks(sGT + col0 * LDZ + k0, LDZ, sF + k0, hi, lo);
        acc = mfma(av, hi, acc);
        acc = mfma(av, lo, acc);
        acc = mfma(frag_cm(sAl + k0 * LDC, LDC), hi, acc);
      }
      // B^T Q[:, block]
      for (int k0 = 0; k0 < C; k0 += 16) {
        bf16x8 hi, lo;
        frag_cm_f32(sBf + k0 * LDF, LDF, hi, lo);
        const bf16x8 b = frag_rm(sQT + col0 * LDC + k0, LDC);
        acc = mfma(hi, b, acc);
        acc = mfma(lo, b, acc);
      }
      // K E_next[:, block]
      for (int k0 = 0; k0 < K; k0 += 16) {
        bf16x8 hi, lo;
        frag_rm_f32(sET + k0, LDE, hi, lo);
        const bf16x8 av = frag_rm(sK + k0, LDK);
        acc = mfma(av, hi, acc);
        acc = mfma(av, lo, acc);
      }
      // in-step suffix of dm
      if (mean) {
        for (int k0 = 0; k0 < C; k0 += 16) {
          bf16x8 hi, lo;
          frag_rm_f32(sDMT + k0, LDF, hi, lo);
          const bf16x8 u1 = frag_triu_ones(0, k0);
          acc = mfma(u1, hi, acc);
          acc = mfma(u1, lo, acc);
        }
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = acc_row(i), c = acc_col();
        if (r < L) {
          const long gi = base + (long)(t0 + r) * rs + col0 + c;
          float d = acc[i] + sDmc[c];
          if (a.dk_extra) d += a.dk_extra[gi];
          if (a.dk) ((bf16*)a.dk)[gi] = (bf16)d;
          if (a.dk32) a.dk32[gi] = d;
        }
      }
    }
    // state: G[:, block] += Q^T dZ[:, block],  Gt[:, block] += dZ^T Q[:, block]
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int rt = w + 4 * j;
      if (rt < NRT) {
        for (int k0 = 0; k0 < C; k0 += 16) {
          const bf16x8 qa = frag_rm(sQT + rt * 32 * LDC + k0, LDC);
          bf16x8 hi, lo;
          frag_rm_f32_ks(sGT + col0 * LDZ + k0, LDZ, sF + k0, hi, lo);
          Gs[j] = mfma(qa, hi, Gs[j]);
          Gs[j] = mfma(qa, lo, Gs[j]);
          bf16x8 ahi, alo;
          frag_rm_f32_ks(sGT + rt * 32 * LDZ + k0, LDZ, sF + k0, ahi, alo);
          const bf16x8 qb = frag_rm(sQT + col0 * LDC + k0, LDC);
          Gt[j] = mfma(ahi, qb, Gt[j]);
          Gt[j] = mfma(alo, qb, Gt[j]);
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int rt = w + 4 * j;
      if (rt < NRT) {
#pragma unroll
        for (int i = 0; i < 16; ++i) sET[acc_col() * LDE + rt * 32 + acc_row(i)] = Gs[j][i] + Gt[j][i];
      }
    }
    if (tid < CB && mean) {
      float s = 0.f;
      for (int r = 0; r < C; ++r) s += sDMT[tid * LDF + r];
      sDmc[tid] += s;
    }
    if (tid < K) sMc[tid] = sMp[tid];
    __syncthreads();
  }

  if (a.dh0) {
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int rt = w + 4 * j;
      if (rt < NRT) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
          a.dh0[((long)unit * K + rt * 32 + acc_row(i)) * K + col0 + acc_col()] = Gs[j][i];
      }
    }
  }
  if (a.dm0 && tid < CB) a.dm0[(long)unit * K + col0 + tid] = mean ? sDmc[tid] : 0.f;
}

// ---------------------------------------------------------------------------
// dlambda reduction over column blocks (+ backward of the fused per-head gate)
// grid (ceil(ntok / 64), H)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void ccq_lam_reduce_kernel(const LamReduceArgs a) {
  __shared__ float sDl[64];
  const int tid = threadIdx.x, h = blockIdx.y;
  const long tok0 = (long)blockIdx.x * 64;
  const int ntk = (int)min((long)64, a.ntok - tok0);
  if (tid < 64) {
    float d = 0.f;
    if (tid < ntk) {
      const long idx = (tok0 + tid) * a.H + h;
      for (int c = 0; c < a.ncb; ++c) d += a.dlam_part[(long)c * a.ntok * a.H + idx];
      if (a.dlam) a.dlam[idx] = d;
      if (a.gate_w) {
        const float lv = a.lam[idx];
        d = d * lv * (1.f - lv);  // dlogit
      }
    }
    sDl[tid] = d;
  }
  __syncthreads();
  if (!a.gate_w) return;
  const int K = a.K;
  const bf16* q = (const bf16*)a.q;
  // dq = dq_clean_path + dlogit W[h];  dW[h] partial = sum_t dlogit_t q_t;  db partial
  for (int kk = tid; kk < K; kk += kThreads) {
    const float wv = a.gate_w[(long)h * K + kk];
    float acc = 0.f;
    for (int t = 0; t < ntk; ++t) {
      const long gi = ((tok0 + t) * a.H + h) * (long)K + kk;
      const float dl = sDl[t];
      acc += dl * (float)q[gi];
      const float d = a.dq32[gi] + dl * wv;
      if (a.dq) ((bf16*)a.dq)[gi] = (bf16)d;
      if (a.dq_out32) a.dq_out32[gi] = d;
    }
    a.dw_part[((long)blockIdx.x * a.H + h) * K + kk] = acc;
  }
  if (tid == 0) {
    float s = 0.f;
    for (int t = 0; t < ntk; ++t) s += sDl[t];
    a.db_part[(long)blockIdx.x * a.H + h] = s;
  }
}

// Sum of `nblk` partial rows: out[j] = sum_b part[b * stride + j], j < cols.
__global__ __launch_bounds__(kThreads) void ccq_sum_rows_kernel(const float* part, float* out, int nblk, int cols) {
  const int j = blockIdx.x * kThreads + threadIdx.x;
  if (j >= cols) return;
  float s = 0.f;
  for (int b = 0; b < nblk; ++b) s += part[(long)b * cols + j];
  out[j] = s;
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
template <int K>
static hipError_t launch_clean_fwd_k(const CleanFwdArgs& a, hipStream_t st) {
  const int grid = (K / kCB) * a.N * a.H;
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL(ccq_clean_fwd_kernel<K>, dim3(grid), dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

template <int K>
static hipError_t launch_clean_bwd_k(const CleanBwdArgs& a, hipStream_t st) {
  const int grid = (K / kCB) * a.N * a.H;
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL(ccq_clean_bwd_kernel<K>, dim3(grid, 2), dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_clean_fwd(const CleanFwdArgs& a, int K, hipStream_t st) {
  switch (K) {
    case 32: return launch_clean_fwd_k<32>(a, st);
    case 64: return launch_clean_fwd_k<64>(a, st);
    case 128: return launch_clean_fwd_k<128>(a, st);
    case 256: return launch_clean_fwd_k<256>(a, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_clean_bwd(const CleanBwdArgs& a, int K, hipStream_t st) {
  switch (K) {
    case 32: return launch_clean_bwd_k<32>(a, st);
    case 64: return launch_clean_bwd_k<64>(a, st);
    case 128: return launch_clean_bwd_k<128>(a, st);
    case 256: return launch_clean_bwd_k<256>(a, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_lam_reduce(const LamReduceArgs& a, hipStream_t st) {
  const int nblk = (int)((a.ntok + 63) / 64);
  if (nblk == 0) return hipSuccess;
  hipLaunchKernelGGL(ccq_lam_reduce_kernel, dim3(nblk, a.H), dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_sum_rows(const float* part, float* out, int nblk, int cols, hipStream_t st) {
  if (cols == 0) return hipSuccess;
  hipLaunchKernelGGL(ccq_sum_rows_kernel, dim3((cols + kThreads - 1) / kThreads), dim3(kThreads), 0, st, part, out,
                     nblk, cols);
  return hipGetLastError();
}

}  // namespace ccq
