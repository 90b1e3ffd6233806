// Cleaning given a precomputed covariance read z (the reference's stock `chunk` path,
// _CCQCleanQ, ccq/ops/common/clean.py:691-748, kernels :220-311 and :405-630), on gfx950.
//
//   m_t = m0 + sum_{j<=t} k_j      s_t = m_t . q_t      pos_t = max(t + 1 + position_offset, 1)
//   corr_t = z_t / pos_t - s_t m_t / pos_t^2      (mean term only with subtract_mean)
//   q_clean_t = q_t - lambda_t corr_t
// Backward (closed form, clean.py:437-445):
//   dz = -lambda dqc / pos;  dlambda = -dqc . corr;  ds = lambda (dqc . m) / pos^2
//   dq = dqc + ds m;         dm_t = ds q_t + lambda s dqc / pos^2
//   dk_j = sum_{t>=j} dm_t (+ dm_final);  dm0 = sum_t dm_t (+ dm_final)
//
// HBM-bound: every kernel streams its rows once.  Tokens are grouped in 64-token blocks per
// (sequence, head); a workgroup of four wavefronts takes one block, each wavefront 16 consecutive
// rows, each lane K/64 channels (channels lane, lane + 64, ...).  The only cross-block quantity is
// the running key sum, carried by a prefix (forward) or suffix (backward) over block totals.
#include "ccq_tile.h"
#include "ccq_zclean_args.h"

namespace ccq {

namespace {

constexpr int BLK = 64;
constexpr int RPW = BLK / 4;  // rows per wavefront

__device__ __forceinline__ bool zc_block(const ZCleanArgs& a, int gb, int& n, int& c0, long& bos, int& L) {
  if (a.cu) {
    n = a.chunk_idx[2 * gb];
    if (n < 0) return false;
    const int c = a.chunk_idx[2 * gb + 1];
    bos = (long)a.cu[n];
    c0 = c * BLK;
    L = min(BLK, (int)(a.cu[n + 1] - a.cu[n]) - c0);
  } else {
    n = gb / a.NT;
    c0 = (gb % a.NT) * BLK;
    bos = (long)n * a.T;
    L = min(BLK, a.T - c0);
  }
  return true;
}

__device__ __forceinline__ float wave_sum(float x) { return group_sum(x, 64); }

}  // namespace

// Column sums of k over each block: ksum[gb][h][:].
template <int K>
__global__ __launch_bounds__(kThreads) void zc_ksum_kernel(const ZCleanArgs a) {
  constexpr int CPL = (K + 63) / 64;
  __shared__ float part[4][K];
  const int w = wave_id(), l = lane_id();
  const int gb = blockIdx.x, h = blockIdx.y;
  int n, c0, L;
  long bos;
  if (!zc_block(a, gb, n, c0, bos, L)) return;
  const long rs = (long)a.H * K;
  float acc[CPL] = {};
  for (int r = w * RPW; r < min(L, (w + 1) * RPW); ++r) {
    const bf16* kr = (const bf16*)a.k + (bos + c0 + r) * rs + (long)h * K;
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      if (l + 64 * j < K) acc[j] += (float)kr[l + 64 * j];
  }
#pragma unroll
  for (int j = 0; j < CPL; ++j)
    if (l + 64 * j < K) part[w][l + 64 * j] = acc[j];
  __syncthreads();
  for (int c = threadIdx.x; c < K; c += kThreads)
    a.ksum[((long)gb * a.H + h) * K + c] = part[0][c] + part[1][c] + part[2][c] + part[3][c];
}

// Per (sequence, head), thread = channel: walk the blocks.
//   DIR 0: prefix[b] = m0 + sum_{b' < b} ksum[b'], m_fin = m0 + sum of all.
//   DIR 1: carry[b] = dm_fin + sum_{b' > b} ksum[b'], dm0 = dm_fin + sum of all.
template <int DIR>
__global__ __launch_bounds__(kThreads) void zc_scan_kernel(const ZCleanArgs a) {
  const int unit = blockIdx.x, c = threadIdx.x;
  if (c >= a.K) return;
  const int n = unit / a.H, h = unit % a.H;
  long bos;
  int len;
  seq_bounds(a.cu, n, a.T, bos, len);
  const int nb = (len + BLK - 1) / BLK;
  const int gb0 = a.cu ? a.chunk_off[n] : n * a.NT;
  const long st = (long)unit * a.K + c;
  if (DIR == 0) {
    float acc = a.m0 ? a.m0[st] : 0.f;
    for (int b = 0; b < nb; ++b) {
      const long o = ((long)(gb0 + b) * a.H + h) * a.K + c;
      a.prefix[o] = acc;
      acc += a.ksum[o];
    }
    if (a.m_fin) a.m_fin[st] = acc;
  } else {
    float acc = a.dm_fin ? a.dm_fin[st] : 0.f;
    for (int b = nb - 1; b >= 0; --b) {
      const long o = ((long)(gb0 + b) * a.H + h) * a.K + c;
      a.carry[o] = acc;
      acc += a.ksum[o];
    }
    if (a.dm0) a.dm0[st] = acc;
  }
}

// Running key sum m_t of this lane's channels for the rows of wavefront w (into mrow[RPW][CPL]).
template <int K, int CPL>
__device__ __forceinline__ void running_sum(const ZCleanArgs& a, long tok0, int h, int L, float (*part)[K],
                                            float (&mrow)[RPW][CPL], int gb) {
  const int w = wave_id(), l = lane_id();
  const long rs = (long)a.H * K;
  float run[CPL] = {};
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int r = w * RPW + i;
    if (r < L) {
      const bf16* kr = (const bf16*)a.k + (tok0 + r) * rs + (long)h * K;
#pragma unroll
      for (int j = 0; j < CPL; ++j)
        if (l + 64 * j < K) run[j] += (float)kr[l + 64 * j];
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) mrow[i][j] = run[j];
  }
#pragma unroll
  for (int j = 0; j < CPL; ++j)
    if (l + 64 * j < K) part[w][l + 64 * j] = run[j];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = l + 64 * j;
    if (c < K) {
      float off = a.prefix[((long)gb * a.H + h) * K + c];
      for (int p = 0; p < w; ++p) off += part[p][c];
#pragma unroll
      for (int i = 0; i < RPW; ++i) mrow[i][j] += off;
    }
  }
}

__device__ __forceinline__ float zc_pos(int t, int off) {
  const float p = (float)(t + 1 + off);
  return p < 1.f ? 1.f : p;
}

template <int K>
__global__ __launch_bounds__(kThreads) void zc_fwd_kernel(const ZCleanArgs a) {
  constexpr int CPL = (K + 63) / 64;
  __shared__ float part[4][K];
  const int w = wave_id(), l = lane_id();
  const int gb = blockIdx.x, h = blockIdx.y;
  int n, c0, L;
  long bos;
  if (!zc_block(a, gb, n, c0, bos, L)) return;
  const long tok0 = bos + c0, rs = (long)a.H * K;
  float mrow[RPW][CPL];
  if (a.subtract_mean) running_sum<K, CPL>(a, tok0, h, L, part, mrow, gb);
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int r = w * RPW + i;
    if (r >= L) break;
    const long off = (tok0 + r) * rs + (long)h * K;
    float q[CPL], z[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const bool ok = l + 64 * j < K;
      q[j] = ok ? (float)((const bf16*)a.q)[off + l + 64 * j] : 0.f;
      z[j] = ok ? (float)((const bf16*)a.z)[off + l + 64 * j] : 0.f;
    }
    const float pos = zc_pos(c0 + r, a.pos_off), ip = 1.f / pos;
    float s = 0.f;
    if (a.subtract_mean) {
#pragma unroll
      for (int j = 0; j < CPL; ++j) s += mrow[i][j] * q[j];
      s = wave_sum(s);
    }
    const float lam = a.lam[(tok0 + r) * a.H + h];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      if (l + 64 * j < K) {
        float corr = z[j] * ip;
        if (a.subtract_mean) corr -= s * ip * ip * mrow[i][j];
        ((bf16*)a.qc)[off + l + 64 * j] = (bf16)(q[j] - lam * corr);
      }
    }
  }
}

// Backward.  PASS 0: block totals of dm (into ksum).  PASS 1: dq, dz, dlambda and dk (suffix of dm
// inside the block + carry of later blocks).
template <int K, int PASS>
__global__ __launch_bounds__(kThreads) void zc_bwd_kernel(const ZCleanArgs a) {
  constexpr int CPL = (K + 63) / 64;
  __shared__ float part[4][K];
  __shared__ float part2[4][K];
  const int w = wave_id(), l = lane_id();
  const int gb = blockIdx.x, h = blockIdx.y;
  int n, c0, L;
  long bos;
  if (!zc_block(a, gb, n, c0, bos, L)) return;
  const long tok0 = bos + c0, rs = (long)a.H * K;
  float mrow[RPW][CPL];
  if (a.subtract_mean) running_sum<K, CPL>(a, tok0, h, L, part, mrow, gb);
  float dmr[RPW][CPL];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int r = w * RPW + i;
#pragma unroll
    for (int j = 0; j < CPL; ++j) dmr[i][j] = 0.f;
    if (r >= L) continue;
    const long off = (tok0 + r) * rs + (long)h * K;
    float q[CPL], z[CPL], g[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const bool ok = l + 64 * j < K;
      const int c = l + 64 * j;
      q[j] = ok ? (float)((const bf16*)a.q)[off + c] : 0.f;
      z[j] = (ok && PASS == 1) ? (float)((const bf16*)a.z)[off + c] : 0.f;
      g[j] = ok ? (a.dqc32 ? a.dqc32[off + c] : (float)((const bf16*)a.dqc16)[off + c]) : 0.f;
    }
    const float pos = zc_pos(c0 + r, a.pos_off), ip = 1.f / pos;
    const float lam = a.lam[(tok0 + r) * a.H + h];
    float s = 0.f, gm = 0.f, ds = 0.f;
    if (a.subtract_mean) {
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        s += mrow[i][j] * q[j];
        gm += mrow[i][j] * g[j];
      }
      s = wave_sum(s);
      gm = wave_sum(gm);
      ds = lam * gm * ip * ip;
#pragma unroll
      for (int j = 0; j < CPL; ++j) dmr[i][j] = ds * q[j] + lam * s * ip * ip * g[j];
    }
    if (PASS == 1) {
      float dl = 0.f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int c = l + 64 * j;
        if (c < K) {
          float corr = z[j] * ip;
          float dq = g[j];
          if (a.subtract_mean) {
            corr -= s * ip * ip * mrow[i][j];
            dq += ds * mrow[i][j];
          }
          dl -= g[j] * corr;
          ((bf16*)a.dq)[off + c] = (bf16)dq;
          ((bf16*)a.dz)[off + c] = (bf16)(-lam * ip * g[j]);
        }
      }
      dl = wave_sum(dl);
      if (l == 0 && a.dlam) a.dlam[(tok0 + r) * a.H + h] = dl;
    }
  }
  // wavefront totals of dm
  float tot[CPL] = {};
#pragma unroll
  for (int i = 0; i < RPW; ++i)
#pragma unroll
    for (int j = 0; j < CPL; ++j) tot[j] += dmr[i][j];
#pragma unroll
  for (int j = 0; j < CPL; ++j)
    if (l + 64 * j < K) part2[w][l + 64 * j] = tot[j];
  __syncthreads();
  if (PASS == 0) {
    for (int c = threadIdx.x; c < K; c += kThreads)
      a.ksum[((long)gb * a.H + h) * K + c] = part2[0][c] + part2[1][c] + part2[2][c] + part2[3][c];
    return;
  }
  // dk_t = sum of dm over rows >= t in the block + later wavefronts + carry of later blocks
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = l + 64 * j;
    if (c >= K) continue;
    float run = a.carry[((long)gb * a.H + h) * K + c];
    for (int p = w + 1; p < 4; ++p) run += part2[p][c];
#pragma unroll
    for (int i = RPW - 1; i >= 0; --i) {
      const int r = w * RPW + i;
      run += dmr[i][j];
      if (r < L) ((bf16*)a.dk)[(tok0 + r) * rs + (long)h * K + c] = (bf16)run;
    }
  }
}

template <int K>
hipError_t launch_zc_k(int stage, const ZCleanArgs& a, hipStream_t st) {
  const dim3 blk(kThreads), grid(a.NB, a.H);
  switch (stage) {
    case 0:  // forward
      hipLaunchKernelGGL(zc_ksum_kernel<K>, grid, blk, 0, st, a);
      hipLaunchKernelGGL(zc_scan_kernel<0>, dim3(a.N * a.H), blk, 0, st, a);
      hipLaunchKernelGGL(zc_fwd_kernel<K>, grid, blk, 0, st, a);
      break;
    case 1:  // backward
      hipLaunchKernelGGL((zc_bwd_kernel<K, 0>), grid, blk, 0, st, a);
      hipLaunchKernelGGL(zc_scan_kernel<1>, dim3(a.N * a.H), blk, 0, st, a);
      hipLaunchKernelGGL((zc_bwd_kernel<K, 1>), grid, blk, 0, st, a);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_zclean(int stage, const ZCleanArgs& a, hipStream_t st) {
  if (a.NB <= 0 || a.H <= 0 || a.N <= 0) return hipSuccess;
  switch (a.K) {
    case 32: return launch_zc_k<32>(stage, a, st);
    case 64: return launch_zc_k<64>(stage, a, st);
    case 128: return launch_zc_k<128>(stage, a, st);
    case 256: return launch_zc_k<256>(stage, a, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ccq
