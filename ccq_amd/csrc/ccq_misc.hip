// Small HBM-bound kernels: row L2 normalisation (forward/backward), the varlen chunk index and
// column sums of partial rows.
#include "ccq_tile.h"
#include "ccq_params.h"

namespace ccq {

// y = x / sqrt(sum x^2 + eps), one 64-lane wavefront per row, element by element (any D <= 512:
// the rows the 16-byte kernels below cannot take).
__global__ __launch_bounds__(kThreads) void l2norm_fwd_kernel(const L2NormArgs a) {
  const long row = (long)blockIdx.x * 4 + wave_id();
  if (row >= a.rows) return;
  const int l = lane_id();
  const bf16* x = (const bf16*)a.x + row * a.D;
  float s = 0.f;
  for (int c = l; c < a.D; c += 64) {
    const float v = (float)x[c];
    s += v * v;
  }
  s = group_sum(s, 64);
  const float r = rsqrtf(s + a.eps);
  bf16* y = (bf16*)a.y + row * a.D;
  for (int c = l; c < a.D; c += 64) y[c] = (bf16)((float)x[c] * r);
  if (l == 0 && a.rstd) a.rstd[row] = r;
}

// dx = r (dy - y (y . dy)),  y = x r  (y recomputed in fp32 from x)
__global__ __launch_bounds__(kThreads) void l2norm_bwd_kernel(const L2NormArgs a) {
  const long row = (long)blockIdx.x * 4 + wave_id();
  if (row >= a.rows) return;
  const int l = lane_id();
  const bf16* x = (const bf16*)a.x + row * a.D;
  const float r = a.rstd[row];
  float s = 0.f;
  for (int c = l; c < a.D; c += 64) {
    const float dy = a.dy32 ? a.dy32[row * a.D + c] : (float)((const bf16*)a.dy16)[row * a.D + c];
    s += (float)x[c] * r * dy;
  }
  s = group_sum(s, 64);
  bf16* dx = (bf16*)a.dx + row * a.D;
  for (int c = l; c < a.D; c += 64) {
    const float dy = a.dy32 ? a.dy32[row * a.D + c] : (float)((const bf16*)a.dy16)[row * a.D + c];
    dx[c] = (bf16)(r * (dy - (float)x[c] * r * s));
  }
}

// The same two passes with 16-byte pieces (D % 8 == 0, 16-byte aligned rows): lr lanes of 8
// consecutive elements per row, 64 / lr rows per wavefront (a row's lanes are one aligned group).
__global__ __launch_bounds__(kThreads) void l2norm_fwd_v_kernel(const L2NormArgs a) {
  const int l = lane_id();
  const long row = ((long)blockIdx.x * 4 + wave_id()) * (64 / a.lr) + l / a.lr;
  if (row >= a.rows) return;  // (whole lane groups)
  const int e = (l & (a.lr - 1)) * 8;
  const bool own = e < a.D;
  float v[8];
  if (own) {
    const bf16x8 xb = *(const bf16x8*)((const bf16*)a.x + row * a.D + e);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (float)xb[i];
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = 0.f;
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += v[i] * v[i];
  s = group_sum(s, a.lr);
  const float r = rsqrtf(s + a.eps);
  if (own) {
    bf16x8 yb;
#pragma unroll
    for (int i = 0; i < 8; ++i) yb[i] = (bf16)(v[i] * r);
    *(bf16x8*)((bf16*)a.y + row * a.D + e) = yb;
  }
  if ((l & (a.lr - 1)) == 0 && a.rstd) a.rstd[row] = r;
}

__global__ __launch_bounds__(kThreads) void l2norm_bwd_v_kernel(const L2NormArgs a) {
  const int l = lane_id();
  const long row = ((long)blockIdx.x * 4 + wave_id()) * (64 / a.lr) + l / a.lr;
  if (row >= a.rows) return;  // (whole lane groups)
  const int e = (l & (a.lr - 1)) * 8;
  const bool own = e < a.D;
  const float r = a.rstd[row];
  float x[8], dy[8];
  if (own) {
    const bf16x8 xb = *(const bf16x8*)((const bf16*)a.x + row * a.D + e);
    if (a.dy32) {
      const f32x4 d0 = *(const f32x4*)(a.dy32 + row * a.D + e), d1 = *(const f32x4*)(a.dy32 + row * a.D + e + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dy[i] = d0[i];
        dy[4 + i] = d1[i];
      }
    } else {
      const bf16x8 db = *(const bf16x8*)((const bf16*)a.dy16 + row * a.D + e);
#pragma unroll
      for (int i = 0; i < 8; ++i) dy[i] = (float)db[i];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = (float)xb[i];
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = dy[i] = 0.f;
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += x[i] * r * dy[i];
  s = group_sum(s, a.lr);
  if (own) {
    bf16x8 o;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (bf16)(r * (dy[i] - x[i] * r * s));
    *(bf16x8*)((bf16*)a.dx + row * a.D + e) = o;
  }
}

// chunk_off[n] = first global `size`-token chunk of sequence n (exclusive scan of ceil(len/size));
// chunk_idx[2c], [2c+1] = (sequence, chunk within sequence) for c < total, -1 beyond it (up to cap).
__global__ __launch_bounds__(kThreads) void chunk_index_kernel(const int64_t* cu, int N, int size, int* chunk_off,
                                                               int* chunk_idx, int cap) {
  __shared__ int sOff[1];
  if (threadIdx.x == 0) {
    int acc = 0;
    for (int n = 0; n < N; ++n) {
      chunk_off[n] = acc;
      const int len = (int)(cu[n + 1] - cu[n]);
      acc += (len + size - 1) / size;
    }
    chunk_off[N] = acc;
    sOff[0] = acc;
  }
  __syncthreads();
  const int total = sOff[0];
  for (int c = threadIdx.x; c < cap; c += kThreads) {
    if (c >= total) {
      chunk_idx[2 * c] = -1;
      chunk_idx[2 * c + 1] = -1;
    }
  }
  // each thread walks a range of sequences
  for (int n = threadIdx.x; n < N; n += kThreads) {
    const int len = (int)(cu[n + 1] - cu[n]);
    const int nc = (len + size - 1) / size;
    const int o = chunk_off[n];
    for (int c = 0; c < nc && o + c < cap; ++c) {
      chunk_idx[2 * (o + c)] = n;
      chunk_idx[2 * (o + c) + 1] = c;
    }
  }
}

// out[i] = 0 for i < n (a kernel rather than hipMemsetAsync, so the call can sit in a captured graph)
__global__ __launch_bounds__(kThreads) void fill_zero_kernel(float* out, long n) {
  for (long i = (long)blockIdx.x * kThreads + threadIdx.x; i < n; i += (long)gridDim.x * kThreads) out[i] = 0.f;
}

hipError_t launch_fill_zero(float* out, long n, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  const long blocks = (n + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)(blocks < 1024 ? blocks : 1024)), dim3(kThreads), 0, st, out, n);
  return hipGetLastError();
}

namespace {
bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// the vector kernels' lanes per row, or 0 where the rows are not whole aligned 16-byte pieces
int l2norm_lanes(const L2NormArgs& a, bool bwd) {
  if (a.D % 8 || !al16(a.x) || !al16(bwd ? a.dx : a.y)) return 0;
  if (bwd && !(a.dy32 ? al16(a.dy32) : al16(a.dy16))) return 0;
  int lr = 1;
  while (lr < 64 && lr * 8 < a.D) lr <<= 1;
  return lr;
}
}  // namespace

hipError_t launch_l2norm_fwd(const L2NormArgs& args, hipStream_t st) {
  if (args.rows == 0) return hipSuccess;
  L2NormArgs a = args;
  a.lr = l2norm_lanes(a, false);
  if (a.lr) {
    const long per = 4L * (64 / a.lr);
    hipLaunchKernelGGL(l2norm_fwd_v_kernel, dim3((unsigned)((a.rows + per - 1) / per)), dim3(kThreads), 0, st, a);
  } else {
    hipLaunchKernelGGL(l2norm_fwd_kernel, dim3((unsigned)((a.rows + 3) / 4)), dim3(kThreads), 0, st, a);
  }
  return hipGetLastError();
}

hipError_t launch_l2norm_bwd(const L2NormArgs& args, hipStream_t st) {
  if (args.rows == 0) return hipSuccess;
  L2NormArgs a = args;
  a.lr = l2norm_lanes(a, true);
  if (a.lr) {
    const long per = 4L * (64 / a.lr);
    hipLaunchKernelGGL(l2norm_bwd_v_kernel, dim3((unsigned)((a.rows + per - 1) / per)), dim3(kThreads), 0, st, a);
  } else {
    hipLaunchKernelGGL(l2norm_bwd_kernel, dim3((unsigned)((a.rows + 3) / 4)), dim3(kThreads), 0, st, a);
  }
  return hipGetLastError();
}

hipError_t launch_chunk_index(const int64_t* cu, int N, int size, int* chunk_off, int* chunk_idx, int cap,
                              hipStream_t st) {
  hipLaunchKernelGGL(chunk_index_kernel, dim3(1), dim3(kThreads), 0, st, cu, N, size, chunk_off, chunk_idx, cap);
  return hipGetLastError();
}

// Two row-sum reductions over the same number of partial rows in one launch per pass (the gate's
// dW [nblk][colsA] and db [nblk][colsB] partials): blocks [0, nbx0) reduce A, the rest B.  Block
// (x, y): 64 columns, rows [y * rps, min(nblk, (y + 1) * rps)); 4 groups of 64 threads.
struct SumRowsPair {
  const float* part[2];
  float* out[2];
  int cols[2];
  int nbx0;
};
__global__ __launch_bounds__(kThreads) void ccq_sum_rows2_kernel(const SumRowsPair p, int nblk, int rps) {
  __shared__ float sP[4][64];
  const int which = blockIdx.x >= (unsigned)p.nbx0 ? 1 : 0;
  const int bx = which ? blockIdx.x - p.nbx0 : blockIdx.x;
  const float* part = which ? p.part[1] : p.part[0];
  float* out = which ? p.out[1] : p.out[0];
  const int cols = which ? p.cols[1] : p.cols[0];
  const int cl = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int j = bx * 64 + cl;
  const int b0 = blockIdx.y * rps, b1 = min(nblk, b0 + rps);
  float s = 0.f;
  if (j < cols)
    for (int b = b0 + grp; b < b1; b += 4) s += part[(long)b * cols + j];
  sP[grp][cl] = s;
  __syncthreads();
  if (grp == 0 && j < cols) out[(long)blockIdx.y * cols + j] = sP[0][cl] + sP[1][cl] + sP[2][cl] + sP[3][cl];
}

// outA[j] = sum_b partA[b * colsA + j] and outB likewise: kSumSlices partial sums over row slices
// [y * rps, (y + 1) * rps) into red[kSumSlices * (colsA + colsB)], then one pass over the slices.
hipError_t launch_sum_rows2(const float* partA, float* outA, int colsA, const float* partB, float* outB, int colsB,
                            int nblk, float* red, hipStream_t st) {
  if (colsA == 0 && colsB == 0) return hipSuccess;
  const int nbA = (colsA + 63) / 64, nbB = (colsB + 63) / 64;
  SumRowsPair p{{partA, partB}, {outA, outB}, {colsA, colsB}, nbA};
  if (nblk <= 4 * kSumSlices || !red) {
    hipLaunchKernelGGL(ccq_sum_rows2_kernel, dim3(nbA + nbB), dim3(kThreads), 0, st, p, nblk, nblk);
    return hipGetLastError();
  }
  const int rps = (nblk + kSumSlices - 1) / kSumSlices;
  const int slices = (nblk + rps - 1) / rps;
  SumRowsPair p1{{partA, partB}, {red, red + (size_t)kSumSlices * colsA}, {colsA, colsB}, nbA};
  hipLaunchKernelGGL(ccq_sum_rows2_kernel, dim3(nbA + nbB, slices), dim3(kThreads), 0, st, p1, nblk, rps);
  SumRowsPair p2{{red, red + (size_t)kSumSlices * colsA}, {outA, outB}, {colsA, colsB}, nbA};
  hipLaunchKernelGGL(ccq_sum_rows2_kernel, dim3(nbA + nbB), dim3(kThreads), 0, st, p2, slices, slices);
  return hipGetLastError();
}

}  // namespace ccq
