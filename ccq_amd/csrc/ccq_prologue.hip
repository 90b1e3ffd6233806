// The layer's prologue and epilogue around the CCQ operators, on gfx950 (reference
// ccq/gdn/layer.py:266-296, 402-408; ccq/gla/layer.py:211-241):
//   short convolution: y = act(bias + sum_w weight[:, w] x[t - (W-1) + w]) per channel (causal,
//                      depthwise, act = SiLU or none), the first W-1 positions of a sequence read
//                      the cached inputs of the previous call; optionally the per-head L2
//                      normalisation of y (yn = y_h / sqrt(|y_h|^2 + eps), computed from y rounded
//                      to bf16, as the operators normalise their bf16 inputs) -- the q / k prologue
//                      in one pass instead of projection -> conv -> SiLU -> l2norm round trips;
//   gated RMSNorm:     y = x / sqrt(mean(x^2) + eps) * weight * silu(g) per row of head_v_dim.
//   narrow linear:     y = x W^T (+ b) with N <= 16 outputs per row (the gate projections
//                      a_proj, b_proj, erase_lambda_proj, gk_proj[0]: ccq/gdn/layer.py:292, 312-316;
//                      ccq/gla/layer.py:162-163) -- a library GEMM tiles N = 4 as it would N = 1024
//                      and spends ~100 us on what is one 34 MB read; here one MFMA pass over x.
// All are HBM-bound streaming passes.  Layout: token-major rows of D channels (bf16); a thread
// owns 8 consecutive channels (one 16-byte piece per row) and walks a tile of tokens; the
// channels of one head are consecutive lanes of one wavefront, so per-head sums are lane
// shuffles.  Weight / bias gradients are per-workgroup partial sums, reduced by a second pass.
#include <algorithm>

#include "ccq_tile.h"
#include "ccq_params.h"

namespace ccq {

namespace {

constexpr int kConvTB = 16;     // tokens per tile of a thread (backward; the forward's is per launch)
constexpr int kDecProMaxH = 32;  // heads of a layer the decode prologue takes

__device__ __forceinline__ float silu_(float a) { return a / (1.f + __expf(-a)); }
__device__ __forceinline__ float dsilu_(float a) {
  const float s = 1.f / (1.f + __expf(-a));
  return s * (1.f + a * (1.f - s));
}

// sum over the `n` consecutive lanes (n a power of two <= 64) that share a head
__device__ __forceinline__ float head_sum(float x, int n) {
  for (int m = 1; m < n; m <<= 1) x += __shfl_xor(x, m);
  return x;
}

// Sequence of packed token p: [start, end) and index.  Dense batches: sequences of T tokens.
struct SeqOf {
  long start, end;
  int n;
};
__device__ __forceinline__ SeqOf seq_of(const ConvArgs& a, long p) {
  SeqOf s;
  if (!a.cu) {
    s.n = (int)(p / a.T);
    s.start = (long)s.n * a.T;
    s.end = s.start + a.T;
    return s;
  }
  int lo = 0, hi = a.N;  // largest n with cu[n] <= p (skipping empty sequences)
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (a.cu[mid] <= p) lo = mid;
    else hi = mid;
  }
  while (lo + 1 < a.N && a.cu[lo + 1] <= p) ++lo;
  s.n = lo;
  s.start = a.cu[lo];
  s.end = a.cu[lo + 1];
  return s;
}

// Eight channels [c, c + 8) of token p: 0 <= p < tokens
__device__ __forceinline__ void load8(const bf16* x, long p, int D, int c, float (&v)[8]) {
  const bf16x8 b = *(const bf16x8*)(x + p * D + c);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (float)b[i];
}

// Input at position rel (relative to its sequence start; rel < 0 reads the cached inputs) of
// sequence sq, channels [c, c + 8).
__device__ __forceinline__ void window_in(const ConvArgs& a, const SeqOf& sq, long rel, int c, float (&v)[8]) {
  if (rel >= 0) {
    load8((const bf16*)a.x, sq.start + rel, a.D, c, v);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      v[i] = a.cache_in ? a.cache_in[((long)sq.n * a.D + c + i) * (a.W - 1) + (a.W - 1) + rel] : 0.f;
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// forward: grid (tiles over the packed tokens (grid-stride), D / 2048), 256 threads
// ---------------------------------------------------------------------------
template <int W>
__global__ __launch_bounds__(kThreads) void conv_fwd_kernel(const ConvArgs a) {
  const int cg = threadIdx.x & (a.cg - 1);
  const long vb = (long)blockIdx.x * (kThreads / a.cg) + threadIdx.x / a.cg;  // this lane's virtual workgroup
  if (vb >= a.nvb) return;  // (whole token lanes: the per-head lane groups stay complete)
  const int c = (blockIdx.y * a.cg + cg) * 8;
  const bool own = c < a.D;
  const int cc = own ? c : 0;
  float wt[8][W], bs[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    bs[i] = a.bias ? a.bias[cc + i] : 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) wt[i][w] = w < W ? a.w[(long)(cc + i) * W + w] : 0.f;
  }
  const int hl = a.hd / 8;  // lanes per head
  const long ntiles = (a.tokens + a.tb - 1) / a.tb;
  for (long tile = vb; tile < ntiles; tile += a.nvb) {
    const long p0 = tile * a.tb, p1 = min(p0 + (long)a.tb, a.tokens);
    SeqOf sq = seq_of(a, p0);
    // window: inputs at positions p - (W-1) .. p - 1 of the current sequence
    float win[W][8];
    auto fill = [&](long p) {
#pragma unroll
      for (int w = 0; w < W - 1; ++w)
        if (w < W - 1) window_in(a, sq, (p - sq.start) - (W - 1) + w, cc, win[w]);
    };
    fill(p0);
    for (long p = p0; p < p1; ++p) {
      if (p >= sq.end) {
        sq = seq_of(a, p);
        fill(p);
      }
      float xv[8];
      load8((const bf16*)a.x, p, a.D, cc, xv);
      float y[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float acc = bs[i] + wt[i][W - 1] * xv[i];
#pragma unroll
        for (int w = 0; w < W - 1; ++w)
          if (w < W - 1) acc += wt[i][w] * win[w][i];
        y[i] = a.act ? silu_(acc) : acc;
      }
      // shift the window
#pragma unroll
      for (int w = 0; w < W - 2; ++w)
        if (w < W - 2)
#pragma unroll
          for (int i = 0; i < 8; ++i) win[w][i] = win[w + 1][i];
      if (W >= 2)
#pragma unroll
        for (int i = 0; i < 8; ++i) win[W - 2][i] = xv[i];
      bf16x8 yb;
#pragma unroll
      for (int i = 0; i < 8; ++i) yb[i] = (bf16)y[i];
      if (own && a.y) *(bf16x8*)((bf16*)a.y + p * a.D + c) = yb;
      if (a.yn) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += (float)yb[i] * (float)yb[i];
        ss = head_sum(own ? ss : 0.f, hl);
        const float r = rsqrtf(ss + a.eps);
        bf16x8 nb;
#pragma unroll
        for (int i = 0; i < 8; ++i) nb[i] = (bf16)((float)yb[i] * r);
        if (own) {
          *(bf16x8*)((bf16*)a.yn + p * a.D + c) = nb;
          if ((threadIdx.x & (hl - 1)) == 0) a.rstd[p * (a.D / a.hd) + c / a.hd] = r;
        }
      }
    }
  }
}

// Final cache: the last W-1 inputs of every sequence (cached inputs of earlier calls for a
// sequence shorter than W-1).  grid (N, ceil(D / 256)).
__global__ __launch_bounds__(kThreads) void conv_cache_kernel(const ConvArgs a) {
  const int n = blockIdx.x, c = blockIdx.y * kThreads + threadIdx.x;
  if (c >= a.D) return;
  const long s0 = a.cu ? a.cu[n] : (long)n * a.T, len = a.cu ? a.cu[n + 1] - a.cu[n] : a.T;
  for (int j = 0; j < a.W - 1; ++j) {
    const long rel = len - (a.W - 1) + j;
    float v;
    if (rel >= 0) v = (float)((const bf16*)a.x)[(s0 + rel) * a.D + c];
    else v = a.cache_in ? a.cache_in[((long)n * a.D + c) * (a.W - 1) + (a.W - 1) + rel] : 0.f;
    a.cache_out[((long)n * a.D + c) * (a.W - 1) + j] = v;
  }
}

// ---------------------------------------------------------------------------
// backward: grid (tiles (grid-stride), D / 2048), 256 threads.  Per token the pre-activation is
// recomputed from x; da = (dy + l2norm backward of dyn) * act'(a); dx[q] = sum_w weight[w] da[q +
// (W-1) - w] over the same sequence; dweight / dbias partials per workgroup.
// ---------------------------------------------------------------------------
template <int W>
__global__ __launch_bounds__(kThreads) void conv_bwd_kernel(const ConvArgs a) {
  const int cg = threadIdx.x & (a.cg - 1);
  const long vb = (long)blockIdx.x * (kThreads / a.cg) + threadIdx.x / a.cg;  // this lane's virtual workgroup
  if (vb >= a.nvb) return;  // (whole token lanes: the per-head lane groups stay complete)
  const int c = (blockIdx.y * a.cg + cg) * 8;
  const bool own = c < a.D;
  const int cc = own ? c : 0;
  float wt[8][W], bs[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    bs[i] = a.bias ? a.bias[cc + i] : 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) wt[i][w] = w < W ? a.w[(long)(cc + i) * W + w] : 0.f;
  }
  float gw[8][W], gb[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    gb[i] = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) gw[i][w] = 0.f;
  }
  const int hl = a.hd / 8;
  const long ntiles = (a.tokens + kConvTB - 1) / kConvTB;
  for (long tile = vb; tile < ntiles; tile += a.nvb) {
    const long p0 = tile * kConvTB, p1 = min(p0 + (long)kConvTB, a.tokens);
    // da of the tokens [p, p + W - 1) after the current one, kept for dx (zero past the sequence)
    float dan[W][8];
#pragma unroll
    for (int w = 0; w < W; ++w)
#pragma unroll
      for (int i = 0; i < 8; ++i) dan[w][i] = 0.f;
    SeqOf sq = seq_of(a, p0);
    float win[W][8];
    auto fill = [&](long p) {
#pragma unroll
      for (int w = 0; w < W - 1; ++w)
        if (w < W - 1) window_in(a, sq, (p - sq.start) - (W - 1) + w, cc, win[w]);
    };
    fill(p0);
    // tokens p0 .. p1 - 1 of the tile plus up to W - 1 more of the last token's sequence
    const SeqOf slast = seq_of(a, p1 - 1);
    const long ptop = min(p1 + (long)(W - 1), slast.end);
    for (long p = p0; p < ptop; ++p) {
      if (p >= sq.end) {
        sq = seq_of(a, p);
        fill(p);
      }
      float xv[8];
      load8((const bf16*)a.x, p, a.D, cc, xv);
      float pre[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float acc = bs[i] + wt[i][W - 1] * xv[i];
#pragma unroll
        for (int w = 0; w < W - 1; ++w)
          if (w < W - 1) acc += wt[i][w] * win[w][i];
        pre[i] = acc;
      }
      // upstream gradient of y at p
      float g[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) g[i] = 0.f;
      if (a.dy) {
        const bf16x8 d = *(const bf16x8*)((const bf16*)a.dy + p * a.D + cc);
#pragma unroll
        for (int i = 0; i < 8; ++i) g[i] = (float)d[i];
      }
      if (a.dyn) {
        // yn = bf16(y) r: dy += r (dyn - yn (yn . dyn)) over the head
        const float r = a.rstd[p * (a.D / a.hd) + cc / a.hd];
        const bf16x8 d = *(const bf16x8*)((const bf16*)a.dyn + p * a.D + cc);
        float yn[8], dot = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float yv = a.act ? silu_(pre[i]) : pre[i];
          yn[i] = (float)(bf16)yv * r;
          dot += yn[i] * (float)d[i];
        }
        dot = head_sum(own ? dot : 0.f, hl);
#pragma unroll
        for (int i = 0; i < 8; ++i) g[i] += r * ((float)d[i] - yn[i] * dot);
      }
      float da[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) da[i] = a.act ? g[i] * dsilu_(pre[i]) : g[i];
      // weight / bias gradients of the tile's own tokens
      if (p < p1) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          gb[i] += da[i];
          gw[i][W - 1] += da[i] * xv[i];
#pragma unroll
          for (int w = 0; w < W - 1; ++w)
            if (w < W - 1) gw[i][w] += da[i] * win[w][i];
        }
      }
      // da of p enters dx of the tokens p - (W-1) .. p of its sequence: shift it in
#pragma unroll
      for (int w = 0; w < W - 1; ++w)
        if (w < W - 1)
#pragma unroll
          for (int i = 0; i < 8; ++i) dan[w][i] = dan[w + 1][i];
#pragma unroll
      for (int i = 0; i < 8; ++i) dan[W - 1][i] = da[i];
      // dx of q = p - (W-1) (dan[j] = da of q + j): sum_w weight[w] da[q + (W-1) - w]
      const long q = p - (W - 1);
      if (q >= p0 && q < p1 && q >= sq.start) {
        bf16x8 o;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float s = 0.f;
#pragma unroll
          for (int w = 0; w < W; ++w)
            if (w < W) s += wt[i][w] * dan[W - 1 - w][i];
          o[i] = (bf16)s;
        }
        if (own) *(bf16x8*)((bf16*)a.dx + q * a.D + c) = o;
      }
      // shift the input window
#pragma unroll
      for (int w = 0; w < W - 2; ++w)
        if (w < W - 2)
#pragma unroll
          for (int i = 0; i < 8; ++i) win[w][i] = win[w + 1][i];
      if (W >= 2)
#pragma unroll
        for (int i = 0; i < 8; ++i) win[W - 2][i] = xv[i];
      // at the end of a sequence, the tile's tokens whose window ran past it get their dx from
      // the da collected so far (the later ones are zero)
      if (p + 1 == sq.end) {
        for (int j = 1; j < W; ++j) {
          const long q2 = p - (W - 1) + j;
          // shift zeros in
#pragma unroll
          for (int w = 0; w < W - 1; ++w)
            if (w < W - 1)
#pragma unroll
              for (int i = 0; i < 8; ++i) dan[w][i] = dan[w + 1][i];
#pragma unroll
          for (int i = 0; i < 8; ++i) dan[W - 1][i] = 0.f;
          if (q2 >= p0 && q2 < p1 && q2 >= sq.start) {
            bf16x8 o;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              float s = 0.f;
#pragma unroll
              for (int w = 0; w < W; ++w)
                if (w < W) s += wt[i][w] * dan[W - 1 - w][i];
              o[i] = (bf16)s;
            }
            if (own) *(bf16x8*)((bf16*)a.dx + q2 * a.D + c) = o;
          }
        }
#pragma unroll
        for (int w = 0; w < W; ++w)
#pragma unroll
          for (int i = 0; i < 8; ++i) dan[w][i] = 0.f;
      }
    }
  }
  // this virtual workgroup's partial sums
  if (own) {
    float* dwp = a.dw_part + vb * a.D * W;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int w = 0; w < W; ++w)
        if (w < W) dwp[(long)(c + i) * W + w] = gw[i][w];
      if (a.db_part) a.db_part[vb * a.D + c + i] = gb[i];
    }
  }
}

// ---------------------------------------------------------------------------
// gated RMSNorm over rows of dv <= 512: lr lanes per row (lane: 8 consecutive elements), 64 / lr
// rows per wavefront, so rows narrower than 512 leave no lane idle
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void gnorm_fwd_kernel(const GNormArgs a) {
  const int l = lane_id(), rpw = 64 / a.lr;
  const long row = ((long)blockIdx.x * 4 + wave_id()) * rpw + l / a.lr;
  if (row >= a.rows) return;  // (whole lane groups: a row's lanes stay together)
  const int e = (l & (a.lr - 1)) * 8;
  const bool own = e < a.dv;
  float x[8], g[8];
  if (own) {
    const bf16x8 xb = *(const bf16x8*)((const bf16*)a.x + row * a.dv + e);
    const bf16x8 gb = *(const bf16x8*)((const bf16*)a.g + (row / a.gper) * a.ldg + (row % a.gper) * a.dv + e);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x[i] = (float)xb[i];
      g[i] = (float)gb[i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = g[i] = 0.f;
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss += x[i] * x[i];
  ss = group_sum(ss, a.lr);
  const float r = rsqrtf(ss / (float)a.dv + a.eps);
  if (own) {
    bf16x8 yb;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float w = a.w ? a.w[e + i] : 1.f;
      yb[i] = (bf16)(x[i] * r * w * silu_(g[i]));
    }
    *(bf16x8*)((bf16*)a.y + row * a.dv + e) = yb;
  }
  if ((l & (a.lr - 1)) == 0) a.rstd[row] = r;
}

// dL/dxh = dy w silu(g); dx = r (dxh - xh mean(dxh xh)); dg = dy xh w silu'(g); dw += dy xh silu(g)
// (partials per workgroup, rows of the grid-stride loop)
__global__ __launch_bounds__(kThreads) void gnorm_bwd_kernel(const GNormArgs a) {
  const int l = lane_id(), rpw = 64 / a.lr, e = (l & (a.lr - 1)) * 8;
  const bool own = e < a.dv;
  float gw[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) gw[i] = 0.f;
  __shared__ float sW[4][512];
  for (long row = ((long)blockIdx.x * 4 + wave_id()) * rpw + l / a.lr; row < a.rows; row += (long)gridDim.x * 4 * rpw) {
    float x[8], g[8], dy[8];
    if (own) {
      const bf16x8 xb = *(const bf16x8*)((const bf16*)a.x + row * a.dv + e);
      const bf16x8 gb = *(const bf16x8*)((const bf16*)a.g + row * a.dv + e);
      const bf16x8 db = *(const bf16x8*)((const bf16*)a.dy + row * a.dv + e);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        x[i] = (float)xb[i];
        g[i] = (float)gb[i];
        dy[i] = (float)db[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = g[i] = dy[i] = 0.f;
    }
    const float r = a.rstd[row];
    float dxh[8], xh[8], dot = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float w = (a.w && own) ? a.w[e + i] : 1.f;
      xh[i] = x[i] * r;
      const float s = silu_(g[i]);
      dxh[i] = dy[i] * w * s;
      dot += dxh[i] * xh[i];
      gw[i] += dy[i] * xh[i] * s;
      g[i] = dy[i] * xh[i] * w * dsilu_(g[i]);  // dg
    }
    dot = group_sum(dot, a.lr) / (float)a.dv;
    if (own) {
      bf16x8 dxb, dgb;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        dxb[i] = (bf16)(r * (dxh[i] - xh[i] * dot));
        dgb[i] = (bf16)g[i];
      }
      *(bf16x8*)((bf16*)a.dx + row * a.dv + e) = dxb;
      *(bf16x8*)((bf16*)a.dg + row * a.dv + e) = dgb;
    }
  }
  if (!a.dw_part) return;
  // the wave's row groups summed by lane swaps (lanes l, l ^ lr, ... hold the same columns), then
  // the workgroup's four waves through LDS, one partial row per workgroup
#pragma unroll
  for (int i = 0; i < 8; ++i)
    for (int m = a.lr; m < 64; m <<= 1) gw[i] += __shfl_xor(gw[i], m);
  if (own && l < a.lr)
#pragma unroll
    for (int i = 0; i < 8; ++i) sW[wave_id()][e + i] = gw[i];
  __syncthreads();
  for (int j = threadIdx.x; j < a.dv; j += kThreads)
    a.dw_part[(long)blockIdx.x * a.dv + j] = sW[0][j] + sW[1][j] + sW[2][j] + sW[3][j];
}

// ---------------------------------------------------------------------------
// decode prologue of a CCQ-GDN layer: grid (B, slices), 256 threads.  Slice 0 takes the q channels
// (all of them: the gate reads the whole q activation), the λ gate and β / g; the next slices take the
// k channels and then the v channels, up to 256 groups of 8 channels each.  A thread owns one group:
// its convolution weights (W 16-byte pieces: the group's [8][W] block), bias and cache window
// ((W-1) 16-byte pieces: the group's [8][W-1] block) are loaded once, the window slides over the
// call's tokens in registers, and the last W-1 inputs go back to the cache from the registers.  The
// lanes of one head are consecutive lanes of one wavefront (K / 8 of them), so the head's sum of
// squares is a lane shuffle in the convolution kernel's order (the same roundings as the layer's
// unfused path: y to bf16, y / sqrt(|y_h|^2 + eps) from the rounded y, to bf16).  The gate's logit
// of head h is the dot product of the whole q activation with row h of its weight: each q thread
// takes its 8 channels against a 16-byte piece of every row, then lane shuffles and one LDS pass.
// ---------------------------------------------------------------------------
template <int W>
__global__ __launch_bounds__(kThreads) void decode_prologue_kernel(const DecProArgs a) {
  __shared__ float sPart[kThreads / 64][kDecProMaxH];
  const int b = blockIdx.x, sl = blockIdx.y, tid = threadIdx.x, l = lane_id(), wv = wave_id();
  const int Dq = a.H * a.K, Dv = a.H * a.V;
  const int nq = Dq / 8, nv = Dv / 8, nks = (nq + kThreads - 1) / kThreads;
  const int hl = a.K / 8;
  int kind, g0, ng, D;
  if (sl == 0) {
    kind = 0; g0 = 0; ng = nq; D = Dq;
  } else if (sl <= nks) {
    kind = 1; g0 = (sl - 1) * kThreads; ng = min(kThreads, nq - g0); D = Dq;
  } else {
    kind = 2; g0 = (sl - 1 - nks) * kThreads; ng = min(kThreads, nv - g0); D = Dv;
  }
  const bool on = tid < ng;
  const int c = 8 * (g0 + (on ? tid : 0));
  const bf16* x = (const bf16*)(kind == 0 ? a.xq : kind == 1 ? a.xk : a.xv);
  const bf16* wt = (const bf16*)(kind == 0 ? a.wq : kind == 1 ? a.wk : a.wv);
  const bf16* bs = (const bf16*)(kind == 0 ? a.bq : kind == 1 ? a.bk : a.bv);
  bf16* cache = (bf16*)(kind == 0 ? a.cq : kind == 1 ? a.ck : a.cv);
  bf16* out = (bf16*)(kind == 0 ? a.q : kind == 1 ? a.k : a.v);

  // the group's weights [8][W], bias, cache window [8][W-1] (in call order: hist[0] the oldest)
  float wgt[8][W], bias[8], hist[W > 1 ? W - 1 : 1][8];
  {
    bf16x8 pw[W];
#pragma unroll
    for (int j = 0; j < W; ++j) pw[j] = *gmem((const bf16x8*)(wt + (long)c * W + 8 * j));
#pragma unroll
    for (int e = 0; e < 8 * W; ++e) wgt[e / W][e % W] = (float)pw[e / 8][e % 8];
    if (bs) {
      const bf16x8 pb = *gmem((const bf16x8*)(bs + c));
#pragma unroll
      for (int i = 0; i < 8; ++i) bias[i] = (float)pb[i];
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) bias[i] = 0.f;
    }
    if constexpr (W > 1) {
      bf16x8 pc[W - 1];
#pragma unroll
      for (int j = 0; j < W - 1; ++j) pc[j] = *gmem((const bf16x8*)(cache + ((long)b * D + c) * (W - 1) + 8 * j));
#pragma unroll
      for (int e = 0; e < 8 * (W - 1); ++e) hist[e % (W - 1)][e / (W - 1)] = (float)pc[e / 8][e % 8];
    }
  }
  // slice 0: the gate weights of this thread's channels, one 16-byte piece per head
  bf16x8 lwp[kDecProMaxH];
  if (kind == 0 && a.lam) {
#pragma unroll
    for (int h = 0; h < kDecProMaxH; ++h)
      if (h < a.H) lwp[h] = *gmem((const bf16x8*)((const bf16*)a.lw + (long)h * Dq + c));
  }

  for (int t = 0; t < a.T; ++t) {
    const long row = (long)b * a.T + t;
    float xv[8];
    {
      const bf16x8 xb = *gmem((const bf16x8*)(x + row * a.ldx + c));
#pragma unroll
      for (int i = 0; i < 8; ++i) xv[i] = (float)xb[i];
    }
    bf16x8 yb;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float acc = bias[i] + wgt[i][W - 1] * xv[i];
#pragma unroll
      for (int w = 0; w < W - 1; ++w) acc += wgt[i][w] * hist[w][i];
      yb[i] = on ? (bf16)silu_(acc) : (bf16)0.f;
    }
    if constexpr (W > 1) {
#pragma unroll
      for (int w = 0; w + 1 < W - 1; ++w)
#pragma unroll
        for (int i = 0; i < 8; ++i) hist[w][i] = hist[w + 1][i];
#pragma unroll
      for (int i = 0; i < 8; ++i) hist[W - 2][i] = xv[i];
    }
    if (kind == 2) {
      if (on) *gmem((bf16x8*)(out + row * Dv + c)) = yb;
      continue;
    }
    // per-head sum of squares (every lane takes part; idle lanes form their own groups)
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += (float)yb[i] * (float)yb[i];
    ss = head_sum(ss, hl);
    const float r = rsqrtf(ss + a.eps);
    bf16x8 nb;
#pragma unroll
    for (int i = 0; i < 8; ++i) nb[i] = (bf16)((float)yb[i] * r);
    if (on) *gmem((bf16x8*)(out + row * Dq + c)) = nb;
    if (kind != 0) continue;
    // gate logits: this thread's channels against every head's weight row, then the workgroup's sum
    // (no lambda output: a layer without cleaning)
#pragma unroll
    for (int h = 0; h < kDecProMaxH; ++h) {
      if (h >= a.H || !a.lam) break;
      float part = 0.f;
      if (on)
#pragma unroll
        for (int i = 0; i < 8; ++i) part += (float)lwp[h][i] * (float)yb[i];
      part = head_sum(part, 64);
      if (l == 0) sPart[wv][h] = part;
    }
    __syncthreads();
    if (tid < a.H) {
      const int h = tid;
      float logit = (a.lb ? (float)((const bf16*)a.lb)[h] : 0.f);
      for (int ww = 0; ww < kThreads / 64; ++ww) logit += sPart[ww][h];
      const float lg = (float)(bf16)logit;                   // the gate projection's bf16 output
      if (a.lam) a.lam[row * a.H + h] = (float)(bf16)(1.f / (1.f + expf(-lg)));
      const float xb = (float)((const bf16*)a.xb)[row * a.ldx + h];
      float be = (float)(bf16)(1.f / (1.f + expf(-xb)));
      if (a.neg_eig) be *= 2.f;
      a.beta[row * a.H + h] = be;
      const float xa = (float)((const bf16*)a.xa)[row * a.ldx + h] + (float)((const bf16*)a.dtb)[h];
      const float sp = xa > 20.f ? xa : log1pf(expf(xa));     // softplus (threshold 20)
      a.g[row * a.H + h] = -expf((float)((const bf16*)a.alog)[h]) * sp;
    }
    __syncthreads();
  }
  // the cache: the last W-1 inputs of the call (or the kept ones, for T < W-1), from the registers
  if constexpr (W > 1) {
    if (on) {
      bf16x8 pc[W - 1];
#pragma unroll
      for (int e = 0; e < 8 * (W - 1); ++e) pc[e / 8][e % 8] = (bf16)hist[e % (W - 1)][e / (W - 1)];
#pragma unroll
      for (int j = 0; j < W - 1; ++j) *gmem((bf16x8*)(cache + ((long)b * D + c) * (W - 1) + 8 * j)) = pc[j];
    }
  }
}

// ===========================================================================
// Narrow linear forward: one wavefront per 16-row tile of x, y[16 x 16] = x[16 x K] W^T[K x 16] by
// 16x16x32 MFMAs with the x fragments loaded straight from HBM (16 bytes per lane, eight steps in
// flight) and W (rows past N zero) in LDS.  Output row r, column n: lane (n, r / 4), element r % 4.
// ===========================================================================
__global__ __launch_bounds__(kThreads) void narrow_fwd_kernel(const NarrowArgs a) {
  extern __shared__ __attribute__((aligned(16))) char narrow_smem[];
  bf16* sw = (bf16*)narrow_smem;  // [16][K + 8]
  const int K = a.K, LDW = K + 8, KV = K / 8;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  for (int idx = tid; idx < 16 * KV; idx += kThreads) {
    const int n = idx / KV, c = (idx % KV) * 8;
    bf16x8 v = bf16x8{};
    if (n < a.N) v = *gmem((const bf16x8*)((const bf16*)a.w + (long)n * K + c));
    *(bf16x8*)(sw + n * LDW + c) = v;
  }
  __syncthreads();
  const long ntile = (a.M + 15) / 16;
  const bf16* wrow = sw + (l & 15) * LDW + 8 * (l >> 4);
  const int n = l & 15;
  const float bn = (a.b && n < a.N) ? a.b[n] : 0.f;
  for (long tile = (long)blockIdx.x * 4 + w; tile < ntile; tile += (long)gridDim.x * 4) {
    const long row = min(tile * 16 + (l & 15), a.M - 1);
    const bf16* xr = (const bf16*)a.x + row * a.ldx + 8 * (l >> 4);
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < K; k0 += 256) {
      bf16x8 xa[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (k0 + 32 * j < K) xa[j] = *gmem((const bf16x8*)(xr + k0 + 32 * j));
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (k0 + 32 * j < K) acc = mfma16(xa[j], *(const bf16x8*)(wrow + k0 + 32 * j), acc);
    }
    if (n < a.N) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const long r = tile * 16 + 4 * (l >> 4) + i;
        if (r < a.M) ((bf16*)a.y)[r * a.N + n] = (bf16)(acc[i] + bn);
      }
    }
  }
}

// ===========================================================================
// Narrow linear backward: a workgroup of roundup64(K / 8) threads takes rpb consecutive rows, a
// thread the same 8 columns of every row.  Per row: dx[8] = sum_n dy[n] W[n][8 cols] (fp32, one
// 16-byte bf16 store), dW[n][8 cols] += dy[n] x[8 cols], db[n] += dy[n] (thread 0).  dy rows are staged
// in LDS 64 at a time (broadcast reads); the block's dW / db go out as one partial row each.
// ===========================================================================
template <int NP>
__global__ __launch_bounds__(kThreads) void narrow_bwd_kernel(const NarrowArgs a) {
  __shared__ float sdy[64][NP];
  const int K = a.K, KV = K / 8;
  const int t = threadIdx.x;
  const bool on = t < KV;
  const int c = (on ? t : 0) * 8;
  bf16x8 wv[NP];
#pragma unroll
  for (int n = 0; n < NP; ++n) wv[n] = (on && n < a.N) ? *gmem((const bf16x8*)((const bf16*)a.w + (long)n * K + c)) : bf16x8{};
  float dw[NP][8], db[NP];
#pragma unroll
  for (int n = 0; n < NP; ++n) {
    db[n] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) dw[n][j] = 0.f;
  }
  const long r0 = (long)blockIdx.x * a.rpb, r1 = min(a.M, r0 + a.rpb);
  for (long rb = r0; rb < r1; rb += 64) {
    const int nr = (int)min(64L, r1 - rb);
    __syncthreads();
    for (int idx = t; idx < 64 * NP; idx += blockDim.x) {
      const int rr = idx / NP, n = idx % NP;
      sdy[rr][n] = (rr < nr && n < a.N) ? (float)((const bf16*)a.dy)[(rb + rr) * a.N + n] : 0.f;
    }
    __syncthreads();
    if (!on) continue;
    for (int rr = 0; rr < nr; ++rr) {
      const long r = rb + rr;
      const bf16x8 xv = *gmem((const bf16x8*)((const bf16*)a.x + r * a.ldx + c));
      float x8[8], d8[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        x8[j] = (float)xv[j];
        d8[j] = 0.f;
      }
#pragma unroll
      for (int n = 0; n < NP; ++n) {
        const float g = sdy[rr][n];
        db[n] += g;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          d8[j] += g * (float)wv[n][j];
          dw[n][j] += g * x8[j];
        }
      }
      if (a.dx) {
        bf16x8 o;
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = (bf16)d8[j];
        *gmem((bf16x8*)((bf16*)a.dx + r * K + c)) = o;
      }
    }
  }
  if (!on) return;
  float* part = a.dw_part + (long)blockIdx.x * a.N * K;
#pragma unroll
  for (int n = 0; n < NP; ++n) {
    if (n < a.N) {
      *gmem((f32x4*)(part + (long)n * K + c)) = f32x4{dw[n][0], dw[n][1], dw[n][2], dw[n][3]};
      *gmem((f32x4*)(part + (long)n * K + c + 4)) = f32x4{dw[n][4], dw[n][5], dw[n][6], dw[n][7]};
    }
  }
  if (a.db_part && t == 0) {
#pragma unroll
    for (int n = 0; n < NP; ++n)
      if (n < a.N) a.db_part[(long)blockIdx.x * a.N + n] = db[n];
  }
}

hipError_t launch_decode_prologue(const DecProArgs& a, hipStream_t st) {
  if (a.B <= 0 || a.T <= 0) return hipSuccess;
  const int nq = a.H * a.K / 8, nv = a.H * a.V / 8;
  if (nq > kThreads) return hipErrorInvalidValue;  // the q slice holds every q channel group
  const dim3 grid((unsigned)a.B, (unsigned)(1 + (nq + kThreads - 1) / kThreads + (nv + kThreads - 1) / kThreads));
  switch (a.W) {
#define CCQ_DECPRO_W(N)                                                        \
  case N:                                                                      \
    hipLaunchKernelGGL(decode_prologue_kernel<N>, grid, dim3(kThreads), 0, st, a); \
    break;
    CCQ_DECPRO_W(1) CCQ_DECPRO_W(2) CCQ_DECPRO_W(3) CCQ_DECPRO_W(4) CCQ_DECPRO_W(5) CCQ_DECPRO_W(6)
    CCQ_DECPRO_W(7) CCQ_DECPRO_W(8)
#undef CCQ_DECPRO_W
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// `blocks` virtual workgroups (the backward's partial rows); each workgroup covers cg groups of 8
// channels (the next power of two of D / 8, at most 256) and 256 / cg token lanes, so narrow
// layers (D / 8 < 256) keep every thread busy instead of leaving the channel groups past D idle.
hipError_t launch_conv(int stage, const ConvArgs& args, int blocks, hipStream_t st) {
  if (args.tokens <= 0 && stage != 2) return hipSuccess;
  ConvArgs a = args;
  int cg = 1;
  while (cg < kThreads && cg * 8 < a.D) cg <<= 1;
  a.cg = cg;
  a.nvb = blocks;
  const int lanes = kThreads / cg;
  const dim3 grid((unsigned)((blocks + lanes - 1) / lanes), (unsigned)((a.D + 8 * cg - 1) / (8 * cg)));
  switch (stage) {
    case 0:
    case 1:
      switch (a.W) {
#define CCQ_CONV_W(N)                                                                      \
  case N:                                                                                  \
    if (stage == 0) hipLaunchKernelGGL(conv_fwd_kernel<N>, grid, dim3(kThreads), 0, st, a); \
    else hipLaunchKernelGGL(conv_bwd_kernel<N>, grid, dim3(kThreads), 0, st, a);             \
    break;
        CCQ_CONV_W(1) CCQ_CONV_W(2) CCQ_CONV_W(3) CCQ_CONV_W(4) CCQ_CONV_W(5) CCQ_CONV_W(6) CCQ_CONV_W(7)
        CCQ_CONV_W(8)
#undef CCQ_CONV_W
        default: return hipErrorInvalidValue;
      }
      break;
    case 2:
      if (a.N > 0 && a.W > 1)
        hipLaunchKernelGGL(conv_cache_kernel, dim3((unsigned)a.N, (unsigned)((a.D + kThreads - 1) / kThreads)),
                           dim3(kThreads), 0, st, a);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Backward blocks of the narrow linear map: 64-row groups, at most kNarrowBlocks partial rows.
int narrow_blocks(long M) { return (int)std::max<long>(1, std::min<long>((M + 63) / 64, kNarrowBlocks)); }

hipError_t launch_narrow(int stage, const NarrowArgs& args, hipStream_t st) {
  if (args.M <= 0) return hipSuccess;
  NarrowArgs a = args;
  if (stage == 0) {
    const long tiles = (a.M + 15) / 16;
    const unsigned grid = (unsigned)std::min<long>((tiles + 3) / 4, 4096);
    const size_t lds = (size_t)16 * (a.K + 8) * sizeof(bf16);
    hipLaunchKernelGGL(narrow_fwd_kernel, dim3(grid), dim3(kThreads), lds, st, a);
    return hipGetLastError();
  }
  const int nb = narrow_blocks(a.M);
  a.rpb = (int)((a.M + nb - 1) / nb);
  const dim3 block((unsigned)(((a.K / 8 + 63) / 64) * 64));
  if (a.N <= 4)
    hipLaunchKernelGGL(narrow_bwd_kernel<4>, dim3(nb), block, 0, st, a);
  else if (a.N <= 8)
    hipLaunchKernelGGL(narrow_bwd_kernel<8>, dim3(nb), block, 0, st, a);
  else
    hipLaunchKernelGGL(narrow_bwd_kernel<16>, dim3(nb), block, 0, st, a);
  return hipGetLastError();
}

hipError_t launch_gnorm(int stage, const GNormArgs& args, int blocks, hipStream_t st) {
  if (args.rows <= 0) return hipSuccess;
  GNormArgs a = args;
  a.lr = 1;
  while (a.lr < 64 && a.lr * 8 < a.dv) a.lr <<= 1;
  const long rows_per_block = 4L * (64 / a.lr);
  if (stage == 0)
    hipLaunchKernelGGL(gnorm_fwd_kernel, dim3((unsigned)((a.rows + rows_per_block - 1) / rows_per_block)),
                       dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL(gnorm_bwd_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

}  // namespace ccq
