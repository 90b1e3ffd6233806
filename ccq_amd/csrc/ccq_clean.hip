// CCQ read-side cleaning operator on gfx950, chunk-parallel form (forward and backward).
//
// Mathematics (per sequence and head; reference ccq/ops/common/fused_read.py:11-25):
//   h_t = h_0 + sum_{j<=t} k_j k_j^T          m_t = m_0 + sum_{j<=t} k_j
//   z_t = h_t^T q_t     s_t = m_t . q_t      corr_t = z_t/pos_t - s_t m_t/pos_t^2
//   q_clean_t = q_t - lambda_t corr_t
//
// The state is a plain (undecayed) running sum, so no kernel walks the sequence.  Tokens are
// grouped in 32-token blocks and 256-token segments:
//   1. segment sums  P_s = sum_{t in s} k_t k_t^T (MFMA), mu_s = sum_{t in s} k_t
//   2. a prefix over the segments of each sequence: H_s = h_0 + sum_{s' < s} P_s', M_s likewise
//   3. one workgroup per block c of segment s:
//        z_t = H_s^T q_t + sum_{key blocks j <= c in s} (Q K_j^T o M) K_j     (causal incl. diagonal)
//        s_t = M_s . q_t + rowsum of the same scores;  cum_t = m_prev + (L1 K_c)_t
//      i.e. causal linear attention over at most eight key blocks plus one state read.
// The backward has the same shape: a dq kernel (queries Q and dZ against the segment's key
// blocks and H_s), a segment sum of q dz^T + dz q^T with a reverse prefix (E after each
// segment), and a dk kernel that runs the transposed attention (query blocks t >= j).
// States enter the MFMAs as hi/lo bf16 pairs, so z (and dlambda = -dqc . corr) keep about
// 16 significant bits even when h_0 dominates.
#include "ccq_tile.h"
#include "ccq_params.h"

namespace ccq {

namespace {

constexpr int kBlk = 32;   // tokens per block
constexpr int kSeg = 256;  // tokens per segment
constexpr int kBps = kSeg / kBlk;

__device__ __forceinline__ void seq_of(const CleanArgs& a, int n, long& bos, int& len) {
  if (a.cu) {
    bos = (long)a.cu[n];
    len = (int)(a.cu[n + 1] - a.cu[n]);
  } else {
    bos = (long)n * a.T;
    len = a.T;
  }
}

// global block id -> (sequence, block); false for padding entries of a varlen launch
__device__ __forceinline__ bool blk_info(const CleanArgs& a, int gb, int& n, int& c) {
  if (a.cu) {
    n = a.blk_idx[2 * gb];
    if (n < 0) return false;
    c = a.blk_idx[2 * gb + 1];
  } else {
    n = gb / a.NB;
    c = gb % a.NB;
  }
  return true;
}

__device__ __forceinline__ bool seg_info(const CleanArgs& a, int gs, int& n, int& s) {
  if (a.cu) {
    n = a.seg_idx[2 * gs];
    if (n < 0) return false;
    s = a.seg_idx[2 * gs + 1];
  } else {
    n = gs / a.NS;
    s = gs % a.NS;
  }
  return true;
}

__device__ __forceinline__ int seg_global(const CleanArgs& a, int n, int s) {
  return a.cu ? a.seg_off[n] + s : n * a.NS + s;
}
__device__ __forceinline__ int blk_global(const CleanArgs& a, int n, int c) {
  return a.cu ? a.blk_off[n] + c : n * a.NB + c;
}

// Workgroups go to the 8 XCDs round-robin by linear id.  The per-block kernels run on a 1-D grid
// of nblk * H workgroups remapped so that each XCD gets a contiguous range of (head, block) pairs,
// block fastest: the eight blocks of a segment then share one XCD's L2 copy of its state.
__device__ __forceinline__ void xcd_blocks(const CleanArgs& a, int& gb, int& h) {
  const int total = gridDim.x, nblk = total / a.H;
  const int q = total >> 3, r = total & 7;
  const int lin = blockIdx.x, xcd = lin & 7, idx = lin >> 3;
  const int m = (xcd < r) ? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
  h = m / nblk;
  gb = m - h * nblk;
}

__device__ __forceinline__ float clamp_pos(int t_local, int off) {
  const float p = (float)(t_local + 1 + off);
  return p < 1.f ? 1.f : p;
}

// Register prefetch of a 32 x D bf16 tile that is stored both row-major and transposed.
// Patches of 4 rows x 8 columns per thread (see stage_bf16_t4).
template <int D>
struct Pre4 {
  static constexpr int RG = kBlk / 4, CG = D / 8, N = (RG * CG + kThreads - 1) / kThreads;
  bf16x8 v[N][4];
  __device__ __forceinline__ void load(const bf16* g, long gstride, int nvalid) {
#pragma unroll
    for (int u = 0; u < N; ++u) {
      const int idx = threadIdx.x + u * kThreads;
      const int rg = idx % RG, cg = idx / RG;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (idx < RG * CG && rg * 4 + j < nvalid) {
          v[u][j] = *(const bf16x8*)(g + (long)(rg * 4 + j) * gstride + cg * 8);
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) v[u][j][i] = (bf16)0.f;
        }
      }
    }
  }
  __device__ __forceinline__ void store(bf16* rows, int ld, bf16* cols, int ldt) const {
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int u = 0; u < N; ++u) {
      const int idx = threadIdx.x + u * kThreads;
      if (idx >= RG * CG) continue;
      const int rg = idx % RG, cg = idx / RG;
      if (rows) {
#pragma unroll
        for (int j = 0; j < 4; ++j) *(bf16x8*)(rows + (rg * 4 + j) * ld + cg * 8) = v[u][j];
      }
      if (cols) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          bf16x4 c;
          c[0] = v[u][0][i];
          c[1] = v[u][1][i];
          c[2] = v[u][2][i];
          c[3] = v[u][3][i];
          *(bf16x4*)(cols + (cg * 8 + i) * ldt + rg * 4) = c;
        }
      }
    }
  }
};

// Register prefetch of rows [r0, r0 + SR) of a K x K bf16 hi/lo state pair; stored into LDS
// with leading dim K + 8.
template <int K, int SR>
struct PreState {
  static constexpr int VPR = K / 8, NV = 2 * SR * VPR, N = (NV + kThreads - 1) / kThreads;
  bf16x8 v[N];
  __device__ __forceinline__ void load(const bf16* ghi, const bf16* glo, int r0) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = threadIdx.x + j * kThreads;
      if (idx < NV) {
        const int which = idx / (SR * VPR), e = idx % (SR * VPR);
        const int r = e / VPR, cc = (e % VPR) * 8;
        v[j] = *(const bf16x8*)((which ? glo : ghi) + (long)(r0 + r) * K + cc);
      }
    }
  }
  __device__ __forceinline__ void store(bf16* hi, bf16* lo) const {
    constexpr int LD = K + 8;
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = threadIdx.x + j * kThreads;
      if (idx < NV) {
        const int which = idx / (SR * VPR), e = idx % (SR * VPR);
        const int r = e / VPR, cc = (e % VPR) * 8;
        *(bf16x8*)((which ? lo : hi) + r * LD + cc) = v[j];
      }
    }
  }
};

// fp32 (dqc32) or bf16 (dqc16) gradient rows into fp32 LDS rows.
template <int K>
__device__ __forceinline__ void stage_grad(float* dst, int ld, const CleanArgs& a, long off, long rs, int nvalid) {
  if (a.dqc32) {
    stage_f32<K>(dst, ld, nullptr, 0, a.dqc32 + off, rs, kBlk, nvalid);
  } else {
    const bf16* g16 = (const bf16*)a.dqc16 + off;
    for (int idx = threadIdx.x; idx < kBlk * (K / 8); idx += kThreads) {
      const int r = idx / (K / 8), c = (idx % (K / 8)) * 8;
      bf16x8 v;
      if (r < nvalid) {
        v = *(const bf16x8*)(g16 + (long)r * rs + c);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (bf16)0.f;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) dst[r * ld + c + i] = (float)v[i];
    }
  }
}

}  // namespace

// ===========================================================================
// 1. segment sums, grid (NSEG, H, K / KC).
//    MODE 0: pseg = sum k k^T, mseg = sum k.   MODE 1: pseg = sum (q dz^T + dz q^T).
//    MODE 2: pseg = sum q dz^T.                 dz_t = -lambda_t dqc_t / pos_t.
// ===========================================================================
template <int K, int MODE>
__global__ __launch_bounds__(kThreads) void clean_segsum_kernel(const CleanArgs a) {
  constexpr int KC = K > 128 ? 128 : K, LDB = kBlk + 8, LDZ = kBlk + 1;
  constexpr int NCT = KC / 32, NT = (K / 32) * NCT, TPW = (NT + 3) / 4;
  __shared__ __attribute__((aligned(16))) bf16 sXT[K * LDB];  // k (MODE 0) or q (MODE 1/2), transposed
  __shared__ float sZT[(MODE == 0) ? 1 : K * LDZ];             // dqc transposed (MODE 1/2)
  __shared__ float sF[kBlk];

  const int tid = threadIdx.x, w = wave_id();
  const int gs = blockIdx.x, h = blockIdx.y, col0 = blockIdx.z * KC;
  int n, s;
  if (!seg_info(a, gs, n, s)) return;
  long bos;
  int len;
  seq_of(a, n, bos, len);
  const long rs = (long)a.H * K;
  const long base = (bos * a.H + h) * (long)K;
  const int tb = s * kSeg, te = min(len, tb + kSeg);
  const bf16* src = (const bf16*)(MODE == 0 ? a.k : a.q) + base;

  f32x16 acc[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) acc[j] = zero16();
  float cs = 0.f;

  for (int t0 = tb; t0 < te; t0 += kBlk) {
    const int L = min(kBlk, te - t0);
    stage_bf16_t4<K, kBlk>(sXT, LDB, src + (long)t0 * rs, rs, L);
    if (MODE != 0) {
      if (tid < kBlk) {
        const float lm = (tid < L) ? a.lam[(bos + t0 + tid) * a.H + h] : 0.f;
        sF[tid] = -lm / clamp_pos(t0 + tid, a.pos_off);
      }
      if (a.dqc32) {
        stage_f32<K>(nullptr, 0, sZT, LDZ, a.dqc32 + base + (long)t0 * rs, rs, kBlk, L);
      } else {
        const bf16* g16 = (const bf16*)a.dqc16 + base + (long)t0 * rs;
        for (int idx = tid; idx < kBlk * K; idx += kThreads) {
          const int r = idx / K, c = idx % K;
          sZT[c * LDZ + r] = (r < L) ? (float)g16[(long)r * rs + c] : 0.f;
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int tile = w + 4 * j;
      if (tile < NT) {
        const int rt = tile / NCT, ct = tile % NCT;
        for (int k0 = 0; k0 < kBlk; k0 += 16) {
          const bf16x8 xa = frag_rm(sXT + rt * 32 * LDB + k0, LDB);
          if (MODE == 0) {
            acc[j] = mfma(xa, frag_rm(sXT + (col0 + ct * 32) * LDB + k0, LDB), acc[j]);
          } else {
            bf16x8 hi, lo;
            frag_rm_f32_ks(sZT + (col0 + ct * 32) * LDZ + k0, LDZ, sF + k0, hi, lo);
            acc[j] = mfma(xa, hi, acc[j]);
            acc[j] = mfma(xa, lo, acc[j]);
            if (MODE == 1) {  // + dz q^T
              bf16x8 zh, zl;
              frag_rm_f32_ks(sZT + rt * 32 * LDZ + k0, LDZ, sF + k0, zh, zl);
              const bf16x8 xb = frag_rm(sXT + (col0 + ct * 32) * LDB + k0, LDB);
              acc[j] = mfma(zh, xb, acc[j]);
              acc[j] = mfma(zl, xb, acc[j]);
            }
          }
        }
      }
    }
    if (MODE == 0 && blockIdx.z == 0 && tid < K) {
      for (int r = 0; r < kBlk; ++r) cs += (float)sXT[tid * LDB + r];
    }
    __syncthreads();
  }
  float* out = a.pseg + ((long)gs * a.H + h) * K * K;
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int tile = w + 4 * j;
    if (tile < NT) {
      const int rt = tile / NCT, ct = tile % NCT;
#pragma unroll
      for (int i = 0; i < 16; ++i) out[(long)(rt * 32 + acc_row(i)) * K + col0 + ct * 32 + acc_col()] = acc[j][i];
    }
  }
  if (MODE == 0 && blockIdx.z == 0 && tid < K) a.mseg[((long)gs * a.H + h) * K + tid] = cs;
}

// ===========================================================================
// 2. prefix over the segments of each (sequence, head), one thread per state element.
//    grid (N * H, ceil(K*K / 256))
//    MODE 0 (forward): hs[s] = (h0 + sum_{s'<s} P_s')^T as hi/lo; h_fin = h0 + sum P
//                      (P is symmetric, so the transpose needs only h0 read transposed).
//    MODE 1 (backward): he[s] = E after segment s = dhf + dhf^T + sum_{s'>s} P_s' (P symmetric).
//    MODE 2 (backward): dh0 = dhf + sum_s P_s  (P = sum q dz^T).
// ===========================================================================
template <int MODE>
__global__ __launch_bounds__(kThreads) void clean_mat_scan_kernel(const CleanArgs a, const int K) {
  const int unit = blockIdx.x, n = unit / a.H, h = unit % a.H;
  const long e = (long)blockIdx.y * kThreads + threadIdx.x;
  if (e >= (long)K * K) return;
  const int r = (int)(e / K), c = (int)(e % K);
  long bos;
  int len;
  seq_of(a, n, bos, len);
  const int ns = (len + kSeg - 1) / kSeg;
  const long KK = (long)K * K;
  if (MODE == 0) {
    float runT = a.h0 ? a.h0[unit * KK + (long)c * K + r] : 0.f;
    float run = a.h0 ? a.h0[unit * KK + e] : 0.f;
    for (int s = 0; s < ns; ++s) {
      const long gi = ((long)seg_global(a, n, s) * a.H + h) * KK + e;
      bf16 hh, ll;
      split2(runT, hh, ll);
      ((bf16*)a.hs_hi)[gi] = hh;
      ((bf16*)a.hs_lo)[gi] = ll;
      const float p = a.pseg[gi];
      runT += p;
      run += p;
    }
    if (a.h_fin) a.h_fin[unit * KK + e] = run;
  } else if (MODE == 1) {
    float run = a.dh_fin ? a.dh_fin[unit * KK + e] + a.dh_fin[unit * KK + (long)c * K + r] : 0.f;
    for (int s = ns - 1; s >= 0; --s) {
      const long gi = ((long)seg_global(a, n, s) * a.H + h) * KK + e;
      bf16 hh, ll;
      split2(run, hh, ll);
      ((bf16*)a.he_hi)[gi] = hh;
      ((bf16*)a.he_lo)[gi] = ll;
      run += a.pseg[gi];
    }
  } else {
    float run = a.dh_fin ? a.dh_fin[unit * KK + e] : 0.f;
    for (int s = 0; s < ns; ++s) run += a.pseg[((long)seg_global(a, n, s) * a.H + h) * KK + e];
    a.dh0[unit * KK + e] = run;
  }
}

// MODE 0: ms[s] = m0 + sum_{s'<s} mseg; m_fin.  MODE 1: carry[b] = dm_fin + sum_{b'>b} dmtot; dm0.
// grid (N * H); thread k < K <= 256
template <int MODE>
__global__ __launch_bounds__(kThreads) void clean_vec_scan_kernel(const CleanArgs a, const int K) {
  const int unit = blockIdx.x, n = unit / a.H, h = unit % a.H, k = threadIdx.x;
  if (k >= K) return;
  long bos;
  int len;
  seq_of(a, n, bos, len);
  if (MODE == 0) {
    const int ns = (len + kSeg - 1) / kSeg;
    float run = a.m0 ? a.m0[(long)unit * K + k] : 0.f;
    for (int s = 0; s < ns; ++s) {
      const long gi = ((long)seg_global(a, n, s) * a.H + h) * K + k;
      a.ms[gi] = run;
      run += a.mseg[gi];
    }
    if (a.m_fin) a.m_fin[(long)unit * K + k] = run;
  } else {
    const int nb = (len + kBlk - 1) / kBlk;
    float run = a.dm_fin ? a.dm_fin[(long)unit * K + k] : 0.f;
    // loads in batches of 8 so they are in flight together (the chain is only the running sum)
    for (int b = nb - 1; b >= 0; b -= 8) {
      float x[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = (b - i >= 0) ? a.dmtot[((long)blk_global(a, n, b - i) * a.H + h) * K + k] : 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (b - i >= 0) a.carry[((long)blk_global(a, n, b - i) * a.H + h) * K + k] = run;
        run += x[i];
      }
    }
    if (a.dm0) a.dm0[(long)unit * K + k] = run;
  }
}

// ===========================================================================
// 3. forward main kernel, grid NBLK * H (see xcd_blocks)
// ===========================================================================
template <int K>
__global__ __launch_bounds__(kThreads) void clean_fwd_main_kernel(const CleanArgs a) {
  constexpr int LDK = K + 8, LDB = kBlk + 8, LDS = kBlk + 1, NCT = K / 32, TPW = (NCT + 3) / 4;
  constexpr int SR = (K > 128) ? 32 : (K < 64 ? K : 64);  // state rows staged at once
  constexpr long kSt = 2L * SR * LDK * 2, kKj = (long)kBlk * LDK * 2 + (long)K * LDB * 2;
  constexpr long kUnion = kSt > kKj ? kSt : kKj;
  __shared__ __attribute__((aligned(16))) bf16 sQ[kBlk * LDK];
  __shared__ __attribute__((aligned(16))) char sU[kUnion];
  __shared__ float sS[kBlk * LDS];
  __shared__ float sM[K];
  __shared__ float sMp[K];
  __shared__ float sW[K];
  __shared__ float sLam[kBlk], sPos[kBlk], sRow[kBlk];
  bf16* sHhi = (bf16*)sU;
  bf16* sHlo = sHhi + SR * LDK;
  bf16* sKj = (bf16*)sU;
  bf16* sKjT = sKj + kBlk * LDK;

  const int tid = threadIdx.x, w = wave_id();
  int gb, h;
  xcd_blocks(a, gb, h);
  int n, c;
  if (!blk_info(a, gb, n, c)) return;
  long bos;
  int len;
  seq_of(a, n, bos, len);
  const long rs = (long)a.H * K;
  const long base = (bos * a.H + h) * (long)K;
  const int t0 = c * kBlk, L = min(kBlk, len - t0);
  const int sidx = t0 / kSeg, cs = sidx * kBps;  // segment and its first block
  const int gs = seg_global(a, n, sidx);
  const bool mean = a.subtract_mean != 0;
  const bf16* kg = (const bf16*)a.k + base;

  const bf16* ghi = (const bf16*)a.hs_hi + ((long)gs * a.H + h) * K * K;
  const bf16* glo = (const bf16*)a.hs_lo + ((long)gs * a.H + h) * K * K;
  PreState<K, SR> pst;  // state rows, one round ahead
  pst.load(ghi, glo, 0);
  stage_bf16<K>(sQ, LDK, nullptr, 0, (const bf16*)a.q + base + (long)t0 * rs, rs, kBlk, L);
  for (int kk = tid; kk < K; kk += kThreads) {
    sM[kk] = mean ? a.ms[((long)gs * a.H + h) * K + kk] : 0.f;
    if (a.gate_w) sW[kk] = a.gate_w[(long)h * K + kk];
  }
  if (tid < kBlk) {
    sPos[tid] = clamp_pos(t0 + tid, a.pos_off);
    if (!a.gate_w) sLam[tid] = (tid < L) ? a.lam[(bos + t0 + tid) * a.H + h] : 0.f;
  }
  Pre4<K> pk;
  pk.load(kg + (long)(cs * kBlk) * rs, rs, min(kBlk, len - cs * kBlk));
  __syncthreads();
  if (a.gate_w) {
    const int r = tid >> 3, part = tid & 7;
    float d = 0.f;
    for (int kk = part; kk < K; kk += 8) d += (float)sQ[r * LDK + kk] * sW[kk];
    d = group_sum(d, 8);
    if (part == 0) {
      const float lv = (r < L) ? sigmoidf_(d + a.gate_b[h]) : 0.f;
      sLam[r] = lv;
      if (a.lam_out && r < L) a.lam_out[(bos + t0 + r) * a.H + h] = lv;
    }
  }

  // Z = Q H_s (the state enters as a hi/lo pair)
  f32x16 Z[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) Z[j] = zero16();
  for (int r0 = 0; r0 < K; r0 += SR) {
    pst.store(sHhi, sHlo);
    __syncthreads();
    if (r0 + SR < K) pst.load(ghi, glo, r0 + SR);
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int ct = w + 4 * j;
      if (ct < NCT && ct * 32 >= r0 && ct * 32 < r0 + SR) {
        mma_rr(Z[j], sQ, LDK, sHhi + (ct * 32 - r0) * LDK, LDK, K);
        mma_rr(Z[j], sQ, LDK, sHlo + (ct * 32 - r0) * LDK, LDK, K);
      }
    }
    __syncthreads();
  }

  // causal attention over the segment's key blocks cs..c
  float rsum = 0.f, mp = 0.f;
  for (int j = cs; j <= c; ++j) {
    pk.store(sKj, LDK, sKjT, LDB);
    __syncthreads();
    if (j < c) pk.load(kg + (long)((j + 1) * kBlk) * rs, rs, min(kBlk, len - (j + 1) * kBlk));
    if (mean && j < c && tid < K) {
      for (int r = 0; r < kBlk; ++r) mp += (float)sKj[r * LDK + tid];
    }
    if (w == 0) {
      f32x16 acc = zero16();
      mma_rr(acc, sQ, LDK, sKj, LDK, K);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = acc_row(i), cc = acc_col();
        sS[r * LDS + cc] = (j < c || cc <= r) ? acc[i] : 0.f;
      }
    }
    __syncthreads();
    if (tid < kBlk) {
      for (int cc = 0; cc < kBlk; ++cc) rsum += sS[tid * LDS + cc];
    }
#pragma unroll
    for (int j2 = 0; j2 < TPW; ++j2) {
      const int ct = w + 4 * j2;
      if (ct < NCT) {
        for (int k0 = 0; k0 < kBlk; k0 += 16) {
          bf16x8 hi, lo;
          frag_rm_f32(sS + k0, LDS, hi, lo);
          const bf16x8 b = frag_rm(sKjT + ct * 32 * LDB + k0, LDB);
          Z[j2] = mfma(hi, b, Z[j2]);
          Z[j2] = mfma(lo, b, Z[j2]);
        }
      }
    }
    if (j < c) __syncthreads();
  }
  if (tid < K) sMp[tid] = sM[tid] + mp;
  if (tid < kBlk) {
    float s = rsum;
    if (mean)
      for (int kk = 0; kk < K; ++kk) s += sM[kk] * (float)sQ[tid * LDK + kk];
    sRow[tid] = s;
  }
  __syncthreads();
  // epilogue: cum = m_prev + L1 K_c  (K_c is the last key block in LDS)
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int ct = w + 4 * j;
    if (ct >= NCT) continue;
    f32x16 cum = zero16();
    if (mean) {
      for (int k0 = 0; k0 < kBlk; k0 += 16)
        cum = mfma(frag_tril_ones(0, k0), frag_rm(sKjT + ct * 32 * LDB + k0, LDB), cum);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = acc_row(i), col = ct * 32 + acc_col();
      if (r < L) {
        const float p = sPos[r];
        float corr = Z[j][i] / p;
        if (mean) corr -= sRow[r] / (p * p) * (sMp[col] + cum[i]);
        const float out = (float)sQ[r * LDK + col] - sLam[r] * corr;
        const long gi = base + (long)(t0 + r) * rs + col;
        if (a.qc) ((bf16*)a.qc)[gi] = (bf16)out;
        if (a.qc32) a.qc32[gi] = out;
      }
    }
  }
}

// ===========================================================================
// 4. backward dq kernel, grid NBLK * H.  With dz_t = F_t dqc_t, F_t = -lambda_t / pos_t:
//   Z = Q H_s + sum_j (Q K_j^T o M) K_j       (z_t, for dlambda = -dqc . corr)
//   Y = dZ H_s + sum_j (dZ K_j^T o M) K_j     (= h_t dz_t)
//   ds_t = -(M_s . dz_t + rowsum(dZ K^T))/pos_t  (= lambda_t (cum_t . dqc_t)/pos_t^2)
//   dq = dqc + ds cum + Y (+ dlogit W[h] for the fused gate)
// Also writes (s_t, ds_t) per token and the per-block sums of dm for the dk kernel.
// ===========================================================================
template <int K>
__global__ __launch_bounds__(kThreads) void clean_bwd_dq_kernel(const CleanArgs a) {
  constexpr int LDK = K + 8, LDG = K + 4, LDB = kBlk + 8, LDS = kBlk + 1, NCT = K / 32, TPW = (NCT + 3) / 4;
  constexpr int SR = (K > 128) ? 32 : (K < 64 ? K : 64);
  constexpr long kSt = 2L * SR * LDK * 2, kKj = (long)kBlk * LDK * 2 + (long)K * LDB * 2;
  constexpr long kUnion = kSt > kKj ? kSt : kKj;
  __shared__ __attribute__((aligned(16))) bf16 sQ[kBlk * LDK];
  __shared__ float sG[kBlk * LDG];  // dqc rows (fp32)
  __shared__ __attribute__((aligned(16))) char sU[kUnion];
  __shared__ float sSA[kBlk * LDS];
  __shared__ float sSB[kBlk * LDS];
  __shared__ float sM[K];
  __shared__ float sMp[K];
  __shared__ float sW[K];
  __shared__ float sLam[kBlk], sPos[kBlk], sF[kBlk], sRow[kBlk], sDS[kBlk], sDl[kBlk];
  __shared__ float sRed[4][kBlk];
  bf16* sHhi = (bf16*)sU;
  bf16* sHlo = sHhi + SR * LDK;
  bf16* sKj = (bf16*)sU;
  bf16* sKjT = sKj + kBlk * LDK;

  const int tid = threadIdx.x, w = wave_id();
  int gb, h;
  xcd_blocks(a, gb, h);
  const bool gate = a.gate_w != nullptr;
  int n, c;
  if (!blk_info(a, gb, n, c)) {
    if (gate) {  // padding block of a varlen launch: its gate partials are zero
      for (int kk = tid; kk < K; kk += kThreads) a.dw_part[((long)gb * a.H + h) * K + kk] = 0.f;
      if (tid == 0) a.db_part[(long)gb * a.H + h] = 0.f;
    }
    return;
  }
  long bos;
  int len;
  seq_of(a, n, bos, len);
  const long rs = (long)a.H * K;
  const long base = (bos * a.H + h) * (long)K;
  const int t0 = c * kBlk, L = min(kBlk, len - t0);
  const int sidx = t0 / kSeg, cs = sidx * kBps;
  const int gs = seg_global(a, n, sidx);
  const bool mean = a.subtract_mean != 0;
  const bf16* kg = (const bf16*)a.k + base;

  const bf16* ghi = (const bf16*)a.hs_hi + ((long)gs * a.H + h) * K * K;
  const bf16* glo = (const bf16*)a.hs_lo + ((long)gs * a.H + h) * K * K;
  PreState<K, SR> pst;  // state rows, one round ahead
  pst.load(ghi, glo, 0);
  stage_bf16<K>(sQ, LDK, nullptr, 0, (const bf16*)a.q + base + (long)t0 * rs, rs, kBlk, L);
  stage_grad<K>(sG, LDG, a, base + (long)t0 * rs, rs, L);
  for (int kk = tid; kk < K; kk += kThreads) {
    sM[kk] = mean ? a.ms[((long)gs * a.H + h) * K + kk] : 0.f;
    if (gate) sW[kk] = a.gate_w[(long)h * K + kk];
  }
  if (tid < kBlk) {
    const float p = clamp_pos(t0 + tid, a.pos_off);
    const float lm = (tid < L) ? a.lam[(bos + t0 + tid) * a.H + h] : 0.f;
    sPos[tid] = p;
    sLam[tid] = lm;
    sF[tid] = -lm / p;
  }
  Pre4<K> pk;
  pk.load(kg + (long)(cs * kBlk) * rs, rs, min(kBlk, len - cs * kBlk));
  __syncthreads();

  f32x16 Z[TPW], Y[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    Z[j] = zero16();
    Y[j] = zero16();
  }
  for (int r0 = 0; r0 < K; r0 += SR) {
    pst.store(sHhi, sHlo);
    __syncthreads();
    if (r0 + SR < K) pst.load(ghi, glo, r0 + SR);
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int ct = w + 4 * j;
      if (ct < NCT && ct * 32 >= r0 && ct * 32 < r0 + SR) {
        const bf16* bh = sHhi + (ct * 32 - r0) * LDK;
        const bf16* bl = sHlo + (ct * 32 - r0) * LDK;
        mma_rr(Z[j], sQ, LDK, bh, LDK, K);
        mma_rr(Z[j], sQ, LDK, bl, LDK, K);
        for (int k0 = 0; k0 < K; k0 += 16) {
          bf16x8 gh, gl;
          frag_rm_f32(sG + k0, LDG, gh, gl);
          const bf16x8 b1 = frag_rm(bh + k0, LDK);
          Y[j] = mfma(gh, b1, Y[j]);
          Y[j] = mfma(gl, b1, Y[j]);
          Y[j] = mfma(gh, frag_rm(bl + k0, LDK), Y[j]);
        }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
#pragma unroll
    for (int i = 0; i < 16; ++i) Y[j][i] *= sF[acc_row(i)];
  }

  float rsA = 0.f, rsB = 0.f, mp = 0.f;
  for (int jb = cs; jb <= c; ++jb) {
    pk.store(sKj, LDK, sKjT, LDB);
    __syncthreads();
    if (jb < c) pk.load(kg + (long)((jb + 1) * kBlk) * rs, rs, min(kBlk, len - (jb + 1) * kBlk));
    if (mean && jb < c && tid < K) {
      for (int r = 0; r < kBlk; ++r) mp += (float)sKj[r * LDK + tid];
    }
    if (w == 0) {
      f32x16 acc = zero16();
      mma_rr(acc, sQ, LDK, sKj, LDK, K);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = acc_row(i), cc = acc_col();
        sSA[r * LDS + cc] = (jb < c || cc <= r) ? acc[i] : 0.f;
      }
    } else if (w == 1) {
      f32x16 acc = zero16();
      for (int k0 = 0; k0 < K; k0 += 16) {
        bf16x8 gh, gl;
        frag_rm_f32(sG + k0, LDG, gh, gl);
        const bf16x8 b = frag_rm(sKj + k0, LDK);
        acc = mfma(gh, b, acc);
        acc = mfma(gl, b, acc);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = acc_row(i), cc = acc_col();
        sSB[r * LDS + cc] = (jb < c || cc <= r) ? sF[r] * acc[i] : 0.f;
      }
    }
    __syncthreads();
    if (tid < kBlk) {
      for (int cc = 0; cc < kBlk; ++cc) {
        rsA += sSA[tid * LDS + cc];
        rsB += sSB[tid * LDS + cc];
      }
    }
#pragma unroll
    for (int j2 = 0; j2 < TPW; ++j2) {
      const int ct = w + 4 * j2;
      if (ct < NCT) {
        for (int k0 = 0; k0 < kBlk; k0 += 16) {
          const bf16x8 b = frag_rm(sKjT + ct * 32 * LDB + k0, LDB);
          bf16x8 hi, lo;
          frag_rm_f32(sSA + k0, LDS, hi, lo);
          Z[j2] = mfma(hi, b, Z[j2]);
          Z[j2] = mfma(lo, b, Z[j2]);
          frag_rm_f32(sSB + k0, LDS, hi, lo);
          Y[j2] = mfma(hi, b, Y[j2]);
          Y[j2] = mfma(lo, b, Y[j2]);
        }
      }
    }
    if (jb < c) __syncthreads();
  }
  if (tid < K) sMp[tid] = sM[tid] + mp;
  if (tid < kBlk) {
    float s = rsA, mg = 0.f;
    if (mean) {
      for (int kk = 0; kk < K; ++kk) {
        s += sM[kk] * (float)sQ[tid * LDK + kk];
        mg += sM[kk] * sG[tid * LDG + kk];
      }
    }
    sRow[tid] = s;
    sDS[tid] = mean ? -(sF[tid] * mg + rsB) / sPos[tid] : 0.f;
  }
  __syncthreads();
  // dlambda = -sum_k dqc corr  (the workgroup holds every column);  cum tiles
  float dlp[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) dlp[i] = 0.f;
  f32x16 CUM[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int ct = w + 4 * j;
    CUM[j] = zero16();
    if (ct >= NCT) continue;
    if (mean) {
      for (int k0 = 0; k0 < kBlk; k0 += 16)
        CUM[j] = mfma(frag_tril_ones(0, k0), frag_rm(sKjT + ct * 32 * LDB + k0, LDB), CUM[j]);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = acc_row(i), col = ct * 32 + acc_col();
      CUM[j][i] += sMp[col];
      const float p = sPos[r];
      float corr = Z[j][i] / p;
      if (mean) corr -= sRow[r] / (p * p) * CUM[j][i];
      dlp[i] += sG[r * LDG + col] * corr;
    }
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    float v = dlp[i];
    for (int m = 1; m < 32; m <<= 1) v += __shfl_xor(v, m);
    dlp[i] = v;
  }
  if ((lane_id() & 31) == 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) sRed[w][acc_row(i)] = dlp[i];
  }
  __syncthreads();
  if (tid < kBlk) {
    const float dl = (tid < L) ? -(sRed[0][tid] + sRed[1][tid] + sRed[2][tid] + sRed[3][tid]) : 0.f;
    const long ti = (bos + t0 + tid) * a.H + h;
    if (tid < L) {
      if (a.dlam) a.dlam[ti] = dl;
      a.sc[2 * ti] = sRow[tid];
      a.sc[2 * ti + 1] = sDS[tid];
    }
    sDl[tid] = gate ? dl * sLam[tid] * (1.f - sLam[tid]) : 0.f;  // dlogit of the fused gate
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int ct = w + 4 * j;
    if (ct >= NCT) continue;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = acc_row(i), col = ct * 32 + acc_col();
      if (r < L) {
        float d = sG[r * LDG + col] + Y[j][i];
        if (mean) d += sDS[r] * CUM[j][i];
        if (gate) d += sDl[r] * sW[col];
        const long gi = base + (long)(t0 + r) * rs + col;
        if (a.dq) ((bf16*)a.dq)[gi] = (bf16)d;
        if (a.dq32) a.dq32[gi] = d;
      }
    }
  }
  const long pb = ((long)gb * a.H + h) * K;
  for (int kk = tid; kk < K; kk += kThreads) {
    if (mean) {
      float dm = 0.f;
      for (int r = 0; r < L; ++r) {
        const float p = sPos[r];
        dm += sLam[r] * sRow[r] / (p * p) * sG[r * LDG + kk] + sDS[r] * (float)sQ[r * LDK + kk];
      }
      a.dmtot[pb + kk] = dm;
    }
    if (gate) {
      float dw = 0.f;
      for (int r = 0; r < L; ++r) dw += sDl[r] * (float)sQ[r * LDK + kk];
      a.dw_part[pb + kk] = dw;
    }
  }
  if (gate && tid == 0) {
    float db = 0.f;
    for (int r = 0; r < L; ++r) db += sDl[r];
    a.db_part[(long)gb * a.H + h] = db;
  }
}

// ===========================================================================
// 5. backward dk kernel, grid NBLK * H.  For the key block j of this workgroup:
//   dk_j = sum_{query blocks t >= j in the segment} [ (K_j dZ_t^T o M) Q_t + (K_j Q_t^T o M) dZ_t ]
//          + K_j E_s + U1 dm_j + carry_j (+ dk_extra)
//   (M keeps t >= j; U1 is the 0/1 upper-triangular matrix: the in-block suffix sum of dm).
// ===========================================================================
template <int K>
__global__ __launch_bounds__(kThreads) void clean_bwd_dk_kernel(const CleanArgs a) {
  constexpr int LDK = K + 8, LDG = K + 4, LDS = kBlk + 1, NCT = K / 32, TPW = (NCT + 3) / 4;
  constexpr int SR = (K > 128) ? 32 : (K < 64 ? K : 64);
  constexpr long kSt = 2L * SR * LDK * 2, kQG = (long)kBlk * LDK * 2 + (long)kBlk * LDG * 4;
  constexpr long kUnion = kSt > kQG ? kSt : kQG;
  __shared__ __attribute__((aligned(16))) bf16 sKj[kBlk * LDK];
  __shared__ __attribute__((aligned(16))) char sU[kUnion];
  __shared__ float sS1[kBlk * LDS];
  __shared__ float sS2[kBlk * LDS];
  __shared__ float sF[kBlk];
  bf16* sEhi = (bf16*)sU;
  bf16* sElo = sEhi + SR * LDK;
  bf16* sQt = (bf16*)sU;
  float* sGt = (float*)(sQt + kBlk * LDK);

  const int tid = threadIdx.x, w = wave_id();
  int gb, h;
  xcd_blocks(a, gb, h);
  int n, c;
  if (!blk_info(a, gb, n, c)) return;
  long bos;
  int len;
  seq_of(a, n, bos, len);
  const long rs = (long)a.H * K;
  const long base = (bos * a.H + h) * (long)K;
  const int t0 = c * kBlk, L = min(kBlk, len - t0);
  const int sidx = t0 / kSeg;
  const int gs = seg_global(a, n, sidx);
  const int nb = (len + kBlk - 1) / kBlk;
  const int ce = min(nb - 1, (sidx + 1) * kBps - 1);  // last block of the segment
  const bool mean = a.subtract_mean != 0;

  const bf16* ehi = (const bf16*)a.he_hi + ((long)gs * a.H + h) * K * K;
  const bf16* elo = (const bf16*)a.he_lo + ((long)gs * a.H + h) * K * K;
  PreState<K, SR> pst;  // E rows, one round ahead
  pst.load(ehi, elo, 0);
  // query block tb (q, dqc, F = -lambda / pos), one block ahead
  PrefetchBf16<K, kBlk> pq;
  PrefetchGrad<K, kBlk> pg;
  float pf = 0.f;
  auto issue_q = [&](int tb) {
    const int tq = tb * kBlk, Lq = min(kBlk, len - tq);
    pq.load((const bf16*)a.q + base + (long)tq * rs, rs, Lq);
    pg.load(a.dqc32 ? a.dqc32 + base + (long)tq * rs : nullptr,
            a.dqc32 ? nullptr : (const bf16*)a.dqc16 + base + (long)tq * rs, rs, Lq);
    if (tid < kBlk) {
      const float lm = (tid < Lq) ? a.lam[(bos + tq + tid) * a.H + h] : 0.f;
      pf = -lm / clamp_pos(tq + tid, a.pos_off);
    }
  };
  issue_q(c);
  stage_bf16<K>(sKj, LDK, nullptr, 0, (const bf16*)a.k + base + (long)t0 * rs, rs, kBlk, L);
  f32x16 D[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) D[j] = zero16();
  for (int r0 = 0; r0 < K; r0 += SR) {
    pst.store(sEhi, sElo);
    __syncthreads();
    if (r0 + SR < K) pst.load(ehi, elo, r0 + SR);
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int ct = w + 4 * j;
      if (ct < NCT && ct * 32 >= r0 && ct * 32 < r0 + SR) {
        mma_rr(D[j], sKj, LDK, sEhi + (ct * 32 - r0) * LDK, LDK, K);
        mma_rr(D[j], sKj, LDK, sElo + (ct * 32 - r0) * LDK, LDK, K);
      }
    }
    __syncthreads();
  }
  for (int tb = c; tb <= ce; ++tb) {
    pq.store(sQt, LDK, nullptr, 0);
    pg.store(a.dqc32 != nullptr, sGt, LDG);
    if (tid < kBlk) sF[tid] = pf;
    __syncthreads();
    if (tb < ce) issue_q(tb + 1);
    // S1[j][t] = k_j . q_t,  S2[j][t] = k_j . dz_t   (t >= j)
    if (w == 0) {
      f32x16 acc = zero16();
      mma_rr(acc, sKj, LDK, sQt, LDK, K);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = acc_row(i), cc = acc_col();
        sS1[r * LDS + cc] = (tb > c || cc >= r) ? acc[i] : 0.f;
      }
    } else if (w == 1) {
      f32x16 acc = zero16();
      for (int k0 = 0; k0 < K; k0 += 16) {
        const bf16x8 av = frag_rm(sKj + k0, LDK);
        bf16x8 gh, gl;
        frag_rm_f32(sGt + k0, LDG, gh, gl);
        acc = mfma(av, gh, acc);
        acc = mfma(av, gl, acc);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = acc_row(i), cc = acc_col();
        sS2[r * LDS + cc] = (tb > c || cc >= r) ? sF[cc] * acc[i] : 0.f;
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int ct = w + 4 * j;
      if (ct >= NCT) continue;
      for (int k0 = 0; k0 < kBlk; k0 += 16) {
        bf16x8 s1h, s1l, zh, zl;
        frag_rm_f32(sS1 + k0, LDS, s1h, s1l);
        frag_cm_f32_ks(sGt + k0 * LDG + ct * 32, LDG, sF + k0, zh, zl);
        D[j] = mfma(s1h, zh, D[j]);
        D[j] = mfma(s1h, zl, D[j]);
        D[j] = mfma(s1l, zh, D[j]);
        bf16x8 s2h, s2l;
        frag_rm_f32(sS2 + k0, LDS, s2h, s2l);
        const bf16x8 qb = frag_cm(sQt + k0 * LDK + ct * 32, LDK);
        D[j] = mfma(s2h, qb, D[j]);
        D[j] = mfma(s2l, qb, D[j]);
      }
    }
    __syncthreads();
  }
  // in-block suffix of dm: dm_t = (lambda_t s_t / pos_t^2) dqc_t + ds_t q_t for this block's rows
  if (mean) {
    stage_bf16<K>(sQt, LDK, nullptr, 0, (const bf16*)a.q + base + (long)t0 * rs, rs, kBlk, L);
    stage_grad<K>(sGt, LDG, a, base + (long)t0 * rs, rs, L);
    if (tid < kBlk) {
      float cg = 0.f, cq = 0.f;
      if (tid < L) {
        const long ti = (bos + t0 + tid) * a.H + h;
        const float p = clamp_pos(t0 + tid, a.pos_off);
        cg = a.lam[ti] * a.sc[2 * ti] / (p * p);
        cq = a.sc[2 * ti + 1];
      }
      sS1[tid] = cg;
      sS2[tid] = cq;
    }
    __syncthreads();
    for (int idx = tid; idx < kBlk * K; idx += kThreads) {
      const int r = idx / K, cc = idx % K;
      sGt[r * LDG + cc] = sS1[r] * sGt[r * LDG + cc] + sS2[r] * (float)sQt[r * LDK + cc];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int ct = w + 4 * j;
      if (ct >= NCT) continue;
      for (int k0 = 0; k0 < kBlk; k0 += 16) {
        bf16x8 hi, lo;
        frag_cm_f32(sGt + k0 * LDG + ct * 32, LDG, hi, lo);
        const bf16x8 u1 = frag_triu_ones(0, k0);
        D[j] = mfma(u1, hi, D[j]);
        D[j] = mfma(u1, lo, D[j]);
      }
    }
  }
  const long pb = ((long)gb * a.H + h) * K;
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int ct = w + 4 * j;
    if (ct >= NCT) continue;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = acc_row(i), col = ct * 32 + acc_col();
      if (r < L) {
        const long gi = base + (long)(t0 + r) * rs + col;
        float d = D[j][i];
        if (mean) d += a.carry[pb + col];
        if (a.dk_extra) d += a.dk_extra[gi];
        if (a.dk) ((bf16*)a.dk)[gi] = (bf16)d;
        if (a.dk32) a.dk32[gi] = d;
      }
    }
  }
}

// Sum of partial rows over a slice: out[y * cols + j] = sum_{b in slice y} part[b * cols + j],
// slice y = rows [y * rps, min(nblk, (y + 1) * rps)).  grid (ceil(cols / 64), slices); 4 groups of 64 threads.
__global__ __launch_bounds__(kThreads) void ccq_sum_rows_kernel(const float* part, float* out, int nblk, int cols,
                                                                int rps) {
  __shared__ float sP[4][64];
  const int cl = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int j = blockIdx.x * 64 + cl;
  const int b0 = blockIdx.y * rps, b1 = min(nblk, b0 + rps);
  float s = 0.f;
  if (j < cols)
    for (int b = b0 + grp; b < b1; b += 4) s += part[(long)b * cols + j];
  sP[grp][cl] = s;
  __syncthreads();
  if (grp == 0 && j < cols) out[(long)blockIdx.y * cols + j] = sP[0][cl] + sP[1][cl] + sP[2][cl] + sP[3][cl];
}

// ===========================================================================
// launchers
// ===========================================================================
namespace {

template <int K>
hipError_t clean_stage_k(int stage, const CleanArgs& a, int nseg, int nblk, hipStream_t st) {
  constexpr int KC = K > 128 ? 128 : K;
  const dim3 scan_grid(a.N * a.H, (K * K + kThreads - 1) / kThreads);
  switch (stage) {
    case kCleanSegsum:
      hipLaunchKernelGGL((clean_segsum_kernel<K, 0>), dim3(nseg, a.H, K / KC), dim3(kThreads), 0, st, a);
      hipLaunchKernelGGL(clean_mat_scan_kernel<0>, scan_grid, dim3(kThreads), 0, st, a, K);
      hipLaunchKernelGGL(clean_vec_scan_kernel<0>, dim3(a.N * a.H), dim3(kThreads), 0, st, a, K);
      break;
    case kCleanFwd:
      hipLaunchKernelGGL(clean_fwd_main_kernel<K>, dim3(nblk * a.H), dim3(kThreads), 0, st, a);
      break;
    case kCleanBwdDq:
      hipLaunchKernelGGL(clean_bwd_dq_kernel<K>, dim3(nblk * a.H), dim3(kThreads), 0, st, a);
      break;
    case kCleanBwdScan:
      hipLaunchKernelGGL((clean_segsum_kernel<K, 1>), dim3(nseg, a.H, K / KC), dim3(kThreads), 0, st, a);
      hipLaunchKernelGGL(clean_mat_scan_kernel<1>, scan_grid, dim3(kThreads), 0, st, a, K);
      hipLaunchKernelGGL(clean_vec_scan_kernel<1>, dim3(a.N * a.H), dim3(kThreads), 0, st, a, K);
      break;
    case kCleanBwdDh0:
      hipLaunchKernelGGL((clean_segsum_kernel<K, 2>), dim3(nseg, a.H, K / KC), dim3(kThreads), 0, st, a);
      hipLaunchKernelGGL(clean_mat_scan_kernel<2>, scan_grid, dim3(kThreads), 0, st, a, K);
      break;
    case kCleanBwdDk:
      hipLaunchKernelGGL(clean_bwd_dk_kernel<K>, dim3(nblk * a.H), dim3(kThreads), 0, st, a);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_clean_stage(int stage, const CleanArgs& a, int K, int nseg, int nblk, hipStream_t st) {
  if (nblk == 0) return hipSuccess;
  switch (K) {
    case 32: return clean_stage_k<32>(stage, a, nseg, nblk, st);
    case 64: return clean_stage_k<64>(stage, a, nseg, nblk, st);
    case 128: return clean_stage_k<128>(stage, a, nseg, nblk, st);
    case 256: return clean_stage_k<256>(stage, a, nseg, nblk, st);
    default: return hipErrorInvalidValue;
  }
}

// out[j] = sum_b part[b * cols + j]: kSumSlices partial sums into red[kSumSlices * cols], then one pass.
hipError_t launch_sum_rows(const float* part, float* out, int nblk, int cols, float* red, hipStream_t st) {
  if (cols == 0) return hipSuccess;
  const dim3 gx((cols + 63) / 64);
  if (nblk <= 4 * kSumSlices || !red) {
    hipLaunchKernelGGL(ccq_sum_rows_kernel, gx, dim3(kThreads), 0, st, part, out, nblk, cols, nblk);
    return hipGetLastError();
  }
  const int rps = (nblk + kSumSlices - 1) / kSumSlices;
  const int slices = (nblk + rps - 1) / rps;
  hipLaunchKernelGGL(ccq_sum_rows_kernel, dim3(gx.x, slices), dim3(kThreads), 0, st, part, red, nblk, cols, rps);
  hipLaunchKernelGGL(ccq_sum_rows_kernel, gx, dim3(kThreads), 0, st, (const float*)red, out, slices, cols, slices);
  return hipGetLastError();
}

}  // namespace ccq
