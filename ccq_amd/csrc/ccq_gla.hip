// Gated linear attention (GLA), chunked (chunk size 64), forward and backward, on gfx950.
//
// Recurrence (arXiv:2312.06635; the backbone the reference calls through fla's chunk_gla,
// ccq/ops/ccq_gla/fused_chunk.py:42-45, ccq/ops/ccq_gla/chunk.py:53-58):
//   S <- diag(exp(gk_t)) S + k_t v_t^T;   o_t = S^T (scale q_t)
// Per chunk, with b the in-chunk cumulative sum of gk (per channel) and b_L its last row:
//   O = scale (Q o e^b) S + A V,   A_ts = scale sum_c q_tc k_sc e^{b_tc - b_sc}  (s <= t)
//   S <- diag(e^{b_L}) S + (K o e^{b_L - b})^T V
// Backward (dS: gradient of the state after the chunk; G: cumulative decay over the sequence):
//   dS_prev = diag(e^{b_L}) dS + (scale Q o e^b)^T dO
//   dq = scale e^b o (dO S^T) + [dA (K o e^{-b})] o e^b,       dA = scale (dO V^T), causal
//   dk = e^{b_L - b} o (V dS^T) + [dA^T (Q o e^b)] o e^{-b}
//   dv = A^T dO + (K o e^{b_L - b}) dS
//   dG_t = q_t o dq_t - k_t o dk_t (+ rowsum(dS_final o S_final) at the last token),
//   dgk = suffix sum of dG over the sequence.
// The pairwise factors e^{b_t - b_s} (s <= t) inside a chunk enter the products split at a
// reference row m, e^{b_t - b_m} e^{b_m - b_s}, with decays gk <= 0:
// * between the two 32-row blocks (t >= 32 > s) at m = 32, where both factors are <= 1: exact
//   for any decay;
// * inside a diagonal 32-row block at its middle row (16, 48, clamped to the last valid row), where
//   a factor is > 1 only across half the block: used while the log decay over each half stays above
//   -kSplitRange in every channel of the wave (e^80 < fp32 max); otherwise that block is formed with
//   one exponential per pair, e^{b_t - b_s} <= 1, as a sum over the channels in fp32.
// So every decay gives a finite result; the per-pair form only costs time in the blocks that need it.
//
// Kernels:
//   gla_intra        chunk-parallel: b (written for the later stages) and A
//   gla_state<0>     one wavefront per (sequence, head, 32 channels, 32 value columns): forward
//                    walk over the chunks, state snapshots (hi/lo bf16) and the final state
//   gla_fwd_o        chunk x 64-column tiles: O
//   gla_state<1>     reverse walk of the state gradient, snapshots and dh0
//   gla_bwd_dv       chunk x 64-column tiles: dv
//   gla_bwd_dqk      chunk x 64-channel slabs: dq, dk, dG and its in-chunk suffix sums
//   gla_gk_carry / gla_gk_add   suffix carry of dG over chunks -> dgk
//
// Precision: operands that are exact bf16 inputs (k, v, dO) enter one MFMA; every operand formed
// in fp32 (decay-scaled q and k, A, dA, the states) enters as a hi/lo bf16 pair, so products keep
// about 16 significant bits.
#include "ccq_tile.h"
#include "ccq_params.h"

namespace ccq {

namespace {

constexpr int BT = 64;
constexpr int KS = 64;            // channel slab of the chunk-parallel kernels
constexpr int LDF = KS + 4;       // fp32 slab row stride (LDS)
constexpr int LDH = 64 + 8;       // bf16 64-wide row stride (LDS)
constexpr float kSplitRange = 80.f;   // largest log factor a split decay may carry (e^80 < fp32 max)

// True when the split of the pairwise decay factors at row m of the 32-row block starting at row
// r0 stays below e^kSplitRange for channel column c of b (rows past L - 1 hold b_{L-1}), in every
// lane of the wave; a NaN range counts as unsafe.
__device__ __forceinline__ bool split_ok(const float* b, int ld, int r0, int m, int L, int c) {
  const int first = min(r0, L - 1), last = min(r0 + 31, L - 1);
  const float bm = b[m * ld + c];
  const float r = fmaxf(b[first * ld + c] - bm, bm - b[last * ld + c]);
  return __ballot(!(r <= kSplitRange)) == 0;
}

__device__ __forceinline__ bool gla_chunk(const GlaArgs& a, int gc, int& n, int& c0, long& bos, int& L) {
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

// 64 rows x 64 columns of fp32 (g32) or bf16 (g16) global rows into fp32 LDS [64][LDF]; rows >= nvalid
// = 0, or (hold_last, fp32 only) a copy of row nvalid - 1 -- for the cumulative decay, which stays at
// its last value past the end of a chunk.
__device__ __forceinline__ void slab_to_f32(float* dst, const float* g32, const bf16* g16, long gstride, int nvalid,
                                            bool hold_last = false) {
  if (g32) {
    for (int idx = threadIdx.x; idx < BT * 16; idx += kThreads) {
      const int r = idx >> 4, c = (idx & 15) * 4;
      f32x4 v;
      if (r < nvalid) v = *(const f32x4*)(g32 + (long)r * gstride + c);
      else if (hold_last) v = *(const f32x4*)(g32 + (long)(nvalid - 1) * gstride + c);
      else v[0] = v[1] = v[2] = v[3] = 0.f;
      *(f32x4*)(dst + r * LDF + c) = v;
    }
  } else {
    for (int idx = threadIdx.x; idx < BT * 8; idx += kThreads) {
      const int r = idx >> 3, c = (idx & 7) * 8;
      bf16x8 v;
      if (r < nvalid) {
        v = *(const bf16x8*)(g16 + (long)r * gstride + c);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (bf16)0.f;
      }
      f32x4 lo4, hi4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lo4[i] = (float)v[i];
        hi4[i] = (float)v[4 + i];
      }
      *(f32x4*)(dst + r * LDF + c) = lo4;
      *(f32x4*)(dst + r * LDF + c + 4) = hi4;
    }
  }
}

// 64 x 64 bf16 tile (rows of a token- or value-major tensor) into LDS [64][LDH], rows >= nvalid = 0.
__device__ __forceinline__ void tile_bf16(bf16* dst, const bf16* g, long gstride, int nvalid) {
  for (int idx = threadIdx.x; idx < BT * 8; idx += kThreads) {
    const int r = idx >> 3, c = (idx & 7) * 8;
    bf16x8 v;
    if (r < nvalid) {
      v = *(const bf16x8*)(g + (long)r * gstride + c);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = (bf16)0.f;
    }
    *(bf16x8*)(dst + r * LDH + c) = v;
  }
}

// Same tile stored transposed: dst[c * LDH + r].
__device__ __forceinline__ void tile_bf16_t(bf16* dst, const bf16* g, long gstride, int nvalid) {
  typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
  for (int idx = threadIdx.x; idx < 16 * 8; idx += kThreads) {
    const int rg = idx & 15, cg = idx >> 4;  // 4-row x 8-column patches
    const int r0 = rg * 4, c0 = cg * 8;
    bf16x8 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (r0 + j < nvalid) {
        v[j] = *(const bf16x8*)(g + (long)(r0 + j) * gstride + c0);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[j][i] = (bf16)0.f;
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      bf16x4 col;
      col[0] = v[0][i];
      col[1] = v[1][i];
      col[2] = v[2][i];
      col[3] = v[3][i];
      *(bf16x4*)(dst + (c0 + i) * LDH + r0) = col;
    }
  }
}

// 64 x 64 fp32 matrix (row stride 64 in global) into LDS [64][65].
__device__ __forceinline__ void mat64_to_lds(float* dst, const float* g) {
  for (int idx = threadIdx.x; idx < BT * 16; idx += kThreads) {
    const int r = idx >> 4, c = (idx & 15) * 4;
    const f32x4 v = *(const f32x4*)(g + r * BT + c);
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[r * (BT + 1) + c + i] = v[i];
  }
}

__device__ __forceinline__ void split8(const float* x, bf16x8& hi, bf16x8& lo) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    bf16 h, l;
    split2(x[i], h, l);
    hi[i] = h;
    lo[i] = l;
  }
}

// acc += (a_hi + a_lo)(b_hi + b_lo), dropping lo x lo
__device__ __forceinline__ void mfma3(f32x16& acc, const bf16x8& ah, const bf16x8& al, const bf16x8& bh,
                                      const bf16x8& bl) {
  acc = mfma(ah, bh, acc);
  acc = mfma(ah, bl, acc);
  acc = mfma(al, bh, acc);
}

}  // namespace

// ===========================================================================
// gla_intra: grid (NTG, H).  b = in-chunk cumsum of gk (to bcum) and A (to a.A).
// Waves 0..2 own the 32x32 blocks (0,0), (1,0), (1,1) of A; the upper block is zero.
// ===========================================================================
template <int K>
__global__ __launch_bounds__(kThreads) void gla_intra_kernel(const GlaArgs a) {
  __shared__ __attribute__((aligned(16))) float sB[BT * LDF];
  __shared__ __attribute__((aligned(16))) float sQ[BT * LDF];
  __shared__ __attribute__((aligned(16))) float sK[BT * LDF];
  __shared__ float sPart[4 * KS];

  const int tid = threadIdx.x, w = wave_id(), l = lane_id();
  const int gc = blockIdx.x, h = blockIdx.y;
  int n, c0, L;
  long bos;
  if (!gla_chunk(a, gc, n, c0, bos, L)) return;
  const long tok0 = bos + c0;
  const long rsk = (long)a.H * K;
  const int I = (w == 0) ? 0 : 1, J = (w == 2) ? 1 : 0;
  // reference row: the block boundary for the off-diagonal block, the middle of a diagonal block
  // (clamped into the valid rows)
  const bool diag = I == J;
  const int mI = diag ? min(32 * I + 16, L - 1) : min(32, L - 1);

  f32x16 acc = zero16();
  for (int s0 = 0; s0 < K; s0 += KS) {
    // b for this slab: column c = tid & 63 over the rows of quarter qr = tid >> 6
    {
      const int c = tid & 63, qr = tid >> 6;
      float run = 0.f, vals[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int t = 16 * qr + j;
        run += (a.gk && t < L) ? a.gk[(tok0 + t) * rsk + (long)h * K + s0 + c] : 0.f;
        vals[j] = run;
      }
      sPart[qr * KS + c] = run;
      __syncthreads();
      float off = 0.f;
      for (int p = 0; p < qr; ++p) off += sPart[p * KS + c];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int t = 16 * qr + j;
        const float b = vals[j] + off;
        sB[t * LDF + c] = b;
        if (t < L) a.bcum[(tok0 + t) * rsk + (long)h * K + s0 + c] = b;
      }
    }
    slab_to_f32(sQ, a.q32 ? a.q32 + tok0 * rsk + (long)h * K + s0 : nullptr,
                a.q32 ? nullptr : (const bf16*)a.q16 + tok0 * rsk + (long)h * K + s0, rsk, L);
    slab_to_f32(sK, nullptr, (const bf16*)a.k + tok0 * rsk + (long)h * K + s0, rsk, L);
    __syncthreads();
    if (w < 3 && (!diag || split_ok(sB, LDF, 32 * I, mI, L, l))) {
      const int r = 32 * I + (l & 31), s = 32 * J + (l & 31);
      for (int k0 = 0; k0 < KS; k0 += 16) {
        const int kb = k0 + ((l >> 5) << 3);
        float xa[8], xb[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int c = kb + i;
          const float bm = sB[mI * LDF + c];
          xa[i] = sQ[r * LDF + c] * __expf(sB[r * LDF + c] - bm);
          xb[i] = sK[s * LDF + c] * __expf(bm - sB[s * LDF + c]);
        }
        bf16x8 ah, al, bh, bl;
        split8(xa, ah, al);
        split8(xb, bh, bl);
        mfma3(acc, ah, al, bh, bl);
      }
    } else if (w < 3) {
      // a diagonal block whose decay is too steep to split: one exponential per pair (<= 1)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int t = 32 * I + acc_row(i), s = 32 * J + acc_col();
        if (s <= t && t < L) {
          float sum = 0.f;
          for (int c = 0; c < KS; ++c)
            sum += sQ[t * LDF + c] * sK[s * LDF + c] * __expf(sB[t * LDF + c] - sB[s * LDF + c]);
          acc[i] += sum;
        }
      }
    }
    __syncthreads();
  }
  float* Ag = a.A + ((long)gc * a.H + h) * (BT * BT);
  if (w < 3) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int t = 32 * I + acc_row(i), s = 32 * J + acc_col();
      Ag[t * BT + s] = (s <= t && t < L) ? a.scale * acc[i] : 0.f;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) Ag[acc_row(i) * BT + 32 + acc_col()] = 0.f;
  }
}

// ===========================================================================
// gla_state<DIR>: grid (N*H * K/32 * V/32), 64 threads (one wavefront per 32x32 state tile).
//   DIR 0: S_next = diag(e^{b_L}) S + (K o e^{b_L - b})^T V, snapshots of S at each chunk start.
//   DIR 1: dS_prev = diag(e^{b_L}) dS + (scale Q o e^b)^T dO, walking backwards, snapshots of dS
//          (the gradient of the state after each chunk).
// Every state element evolves independently (diagonal decay), so tiles never exchange data.
// Lane l holds token l of the chunk; it writes its rows of the operands as 16-byte pieces
// ([token][column], row-major) and the MFMAs read them with transposing LDS reads.
// ===========================================================================
template <int DIR>
__global__ __launch_bounds__(64) void gla_state_kernel(const GlaArgs a) {
  constexpr int LDR = 32 + 8;  // bank-conflict-free 16-byte row writes, 8-byte aligned transposing reads
  __shared__ __attribute__((aligned(16))) bf16 sXh[BT * LDR];  // A operand rows [token][channel], hi
  __shared__ __attribute__((aligned(16))) bf16 sXl[BT * LDR];  // lo
  __shared__ __attribute__((aligned(16))) bf16 sY[BT * LDR];   // B operand rows [token][value col]
  __shared__ float sBL[32];

  const int l = threadIdx.x;
  const int K = a.K, V = a.V;
  const int nct = K / 32, nvt = V / 32;
  int unit, split;
  xcd_map(blockIdx.x, nct * nvt, a.N * a.H, unit, split);
  const int ct = split % nct, vt = split / nct;
  const int n = unit / a.H, h = unit % a.H;
  const int cb = ct * 32, vb = vt * 32;
  long bos;
  int len;
  seq_bounds(a.cu, n, a.T, bos, len);
  const int nc = (len + BT - 1) / BT;
  const int gc0 = a.cu ? a.chunk_off[n] : n * a.NT;
  const long rsk = (long)a.H * K, rsv = (long)a.H * V;

  f32x16 S;
  {
    const float* init = DIR == 0 ? a.h0 : a.ds_fin;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      S[i] = init ? init[((long)unit * K + cb + acc_row(i)) * V + vb + acc_col()] : 0.f;
  }

  // Row l (token) of the chunk, one step ahead: x (k or q), b, y (v or dO), 32 columns each.
  bf16x8 px[4], py[4];
  f32x4 pq[8], pb[8];
  auto issue = [&](int c) {
    const int L = min(BT, len - c * BT);
    const long tok = bos + (long)c * BT + l;
    const bool ok = l < L;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (ok) pb[j] = *(const f32x4*)(a.bcum + tok * rsk + (long)h * K + cb + 4 * j);
      else pb[j][0] = pb[j][1] = pb[j][2] = pb[j][3] = 0.f;
    }
    const bool xf32 = DIR == 1 && a.q32 != nullptr;
    if (xf32) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (ok) pq[j] = *(const f32x4*)(a.q32 + tok * rsk + (long)h * K + cb + 4 * j);
        else pq[j][0] = pq[j][1] = pq[j][2] = pq[j][3] = 0.f;
      }
    } else {
      const bf16* xs = DIR == 0 ? (const bf16*)a.k : (const bf16*)a.q16;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (ok) {
          px[j] = *(const bf16x8*)(xs + tok * rsk + (long)h * K + cb + 8 * j);
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) px[j][i] = (bf16)0.f;
        }
      }
    }
    const bf16* ys = DIR == 0 ? (const bf16*)a.v : (const bf16*)a.dout;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (ok) {
        py[j] = *(const bf16x8*)(ys + tok * rsv + (long)h * V + vb + 8 * j);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) py[j][i] = (bf16)0.f;
      }
    }
  };

  if (nc > 0) issue(DIR == 0 ? 0 : nc - 1);
  for (int step = 0; step < nc; ++step) {
    const int c = DIR == 0 ? step : nc - 1 - step;
    const int L = min(BT, len - c * BT);
    const int gc = gc0 + c;
    if (l == L - 1) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
#pragma unroll
        for (int i = 0; i < 4; ++i) sBL[4 * j + i] = pb[j][i];
      }
    }
    __syncthreads();
    const bool xf32 = DIR == 1 && a.q32 != nullptr;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      bf16x8 xh, xl;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int cc = 8 * j + i;
        const float bt = pb[cc >> 2][cc & 3];
        const float xv = xf32 ? pq[cc >> 2][cc & 3] : (float)px[j][i];
        const float val = DIR == 0 ? xv * __expf(sBL[cc] - bt) : a.scale * xv * __expf(bt);
        bf16 hh, ll;
        split2(val, hh, ll);
        xh[i] = hh;
        xl[i] = ll;
      }
      *(bf16x8*)(sXh + l * LDR + 8 * j) = xh;
      *(bf16x8*)(sXl + l * LDR + 8 * j) = xl;
      *(bf16x8*)(sY + l * LDR + 8 * j) = py[j];
    }
    float dec[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) dec[i] = __expf(sBL[acc_row(i)]);
    __syncthreads();
    if (step + 1 < nc) issue(DIR == 0 ? c + 1 : c - 1);
    // snapshot of the current (gradient) state, transposed [v][c], as hi/lo bf16
    {
      typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
      bf16* dh = (bf16*)(DIR == 0 ? a.hT : a.dhT);
      bf16* dl = (bf16*)(DIR == 0 ? a.hTl : a.dhTl);
      const long base = (((long)gc * a.H + h) * V + vb + acc_col()) * K + cb;
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        bf16x4 vh, vl;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          bf16 hh, ll;
          split2(S[4 * g4 + i], hh, ll);
          vh[i] = hh;
          vl[i] = ll;
        }
        const int r0 = acc_row(4 * g4);
        *(bf16x4*)(dh + base + r0) = vh;
        *(bf16x4*)(dl + base + r0) = vl;
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) S[i] *= dec[i];
#pragma unroll
    for (int k0 = 0; k0 < BT; k0 += 16) {
      const bf16x8 ah = frag32_tr(sXh + k0 * LDR, LDR);
      const bf16x8 al = frag32_tr(sXl + k0 * LDR, LDR);
      const bf16x8 b = frag32_tr(sY + k0 * LDR, LDR);
      S = mfma(ah, b, S);
      S = mfma(al, b, S);
    }
    __syncthreads();
  }
  float* out = DIR == 0 ? a.s_fin : a.dh0;
  if (out) {
#pragma unroll
    for (int i = 0; i < 16; ++i) out[((long)unit * K + cb + acc_row(i)) * V + vb + acc_col()] = S[i];
  }
}

// ===========================================================================
// gla_fwd_o: grid NTG * H * (V/64), XCD-mapped.  O[:, tile] = scale (Q o e^b) S[:, tile] + A V[:, tile]
// ===========================================================================
template <int K>
__global__ __launch_bounds__(kThreads) void gla_fwd_o_kernel(const GlaArgs a) {
  __shared__ __attribute__((aligned(16))) float sQ[BT * LDF];  // scale q e^b, one slab
  __shared__ __attribute__((aligned(16))) float sBb[BT * LDF];
  __shared__ __attribute__((aligned(16))) bf16 sSh[64 * LDH];  // S piece [v][c] hi
  __shared__ __attribute__((aligned(16))) bf16 sSl[64 * LDH];
  __shared__ __attribute__((aligned(16))) float sA[BT * (BT + 1)];
  __shared__ __attribute__((aligned(16))) bf16 sVt[64 * LDH];  // V tile [v][s]

  const int tid = threadIdx.x, w = wave_id();
  // the V / 64 value blocks of a (chunk, head) unit share its operands: one XCD (L2) per unit
  int unit, vb;
  xcd_map(blockIdx.x, a.V / 64, a.NTG * a.H, unit, vb);
  const int gc = unit / a.H, h = unit % a.H, v0 = vb * 64;
  int n, c0, L;
  long bos;
  if (!gla_chunk(a, gc, n, c0, bos, L)) return;
  const long tok0 = bos + c0;
  const long rsk = (long)a.H * K, rsv = (long)a.H * a.V;
  const int tr = w >> 1, tc = w & 1;

  mat64_to_lds(sA, a.A + ((long)gc * a.H + h) * (BT * BT));
  tile_bf16_t(sVt, (const bf16*)a.v + tok0 * rsv + (long)h * a.V + v0, rsv, L);

  f32x16 acc = zero16();
  const long sbase = (((long)gc * a.H + h) * a.V + v0) * K;
  for (int s0 = 0; s0 < K; s0 += KS) {
    slab_to_f32(sQ, a.q32 ? a.q32 + tok0 * rsk + (long)h * K + s0 : nullptr,
                a.q32 ? nullptr : (const bf16*)a.q16 + tok0 * rsk + (long)h * K + s0, rsk, L);
    slab_to_f32(sBb, a.bcum + tok0 * rsk + (long)h * K + s0, nullptr, rsk, L);
    tile_bf16(sSh, (const bf16*)a.hT + sbase + s0, K, 64);
    tile_bf16(sSl, (const bf16*)a.hTl + sbase + s0, K, 64);
    __syncthreads();
    for (int e = tid; e < BT * KS; e += kThreads) {
      const int r = e >> 6, c = e & 63;
      sQ[r * LDF + c] = a.scale * sQ[r * LDF + c] * __expf(sBb[r * LDF + c]);
    }
    __syncthreads();
    for (int k0 = 0; k0 < KS; k0 += 16) {
      bf16x8 ah, al;
      frag_rm_f32(sQ + tr * 32 * LDF + k0, LDF, ah, al);
      const bf16x8 bh = frag_rm(sSh + tc * 32 * LDH + k0, LDH);
      const bf16x8 bl = frag_rm(sSl + tc * 32 * LDH + k0, LDH);
      mfma3(acc, ah, al, bh, bl);
    }
    __syncthreads();
  }
  for (int k0 = 0; k0 < BT; k0 += 16) {
    bf16x8 ah, al;
    frag_rm_f32(sA + tr * 32 * (BT + 1) + k0, BT + 1, ah, al);
    const bf16x8 b = frag_rm(sVt + tc * 32 * LDH + k0, LDH);
    acc = mfma(ah, b, acc);
    acc = mfma(al, b, acc);
  }
  bf16* og = (bf16*)a.o + tok0 * rsv + (long)h * a.V + v0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = tr * 32 + acc_row(i);
    if (r < L) og[(long)r * rsv + tc * 32 + acc_col()] = (bf16)acc[i];
  }
}

// ===========================================================================
// gla_bwd_dv: grid NTG * H * (V/64), XCD-mapped.  dv[:, tile] = A^T dO[:, tile] + (K o e^{b_L - b}) dS[:, tile]
// ===========================================================================
template <int K>
__global__ __launch_bounds__(kThreads) void gla_bwd_dv_kernel(const GlaArgs a) {
  __shared__ __attribute__((aligned(16))) float sKt[BT * LDF];  // k e^{b_L - b}, one slab
  __shared__ __attribute__((aligned(16))) float sBb[BT * LDF];
  __shared__ __attribute__((aligned(16))) bf16 sDh[64 * LDH];   // dS piece [v][c] hi
  __shared__ __attribute__((aligned(16))) bf16 sDl[64 * LDH];
  __shared__ __attribute__((aligned(16))) float sA[BT * (BT + 1)];
  __shared__ __attribute__((aligned(16))) bf16 sOt[64 * LDH];   // dO tile [v][t]

  const int tid = threadIdx.x, w = wave_id();
  // the V / 64 value blocks of a (chunk, head) unit share its operands: one XCD (L2) per unit
  int unit, vb;
  xcd_map(blockIdx.x, a.V / 64, a.NTG * a.H, unit, vb);
  const int gc = unit / a.H, h = unit % a.H, v0 = vb * 64;
  int n, c0, L;
  long bos;
  if (!gla_chunk(a, gc, n, c0, bos, L)) return;
  const long tok0 = bos + c0;
  const long rsk = (long)a.H * K, rsv = (long)a.H * a.V;
  const int tr = w >> 1, tc = w & 1;

  mat64_to_lds(sA, a.A + ((long)gc * a.H + h) * (BT * BT));
  tile_bf16_t(sOt, (const bf16*)a.dout + tok0 * rsv + (long)h * a.V + v0, rsv, L);
  __syncthreads();

  f32x16 acc = zero16();
  // A^T dO: operand (s, t) = A[t][s]
  for (int k0 = 0; k0 < BT; k0 += 16) {
    bf16x8 ah, al;
    frag_cm_f32(sA + tr * 32 + k0 * (BT + 1), BT + 1, ah, al);
    const bf16x8 b = frag_rm(sOt + tc * 32 * LDH + k0, LDH);
    acc = mfma(ah, b, acc);
    acc = mfma(al, b, acc);
  }
  const long sbase = (((long)gc * a.H + h) * a.V + v0) * K;
  for (int s0 = 0; s0 < K; s0 += KS) {
    slab_to_f32(sKt, nullptr, (const bf16*)a.k + tok0 * rsk + (long)h * K + s0, rsk, L);
    slab_to_f32(sBb, a.bcum + tok0 * rsk + (long)h * K + s0, nullptr, rsk, L);
    tile_bf16(sDh, (const bf16*)a.dhT + sbase + s0, K, 64);
    tile_bf16(sDl, (const bf16*)a.dhTl + sbase + s0, K, 64);
    __syncthreads();
    for (int e = tid; e < BT * KS; e += kThreads) {
      const int r = e >> 6, c = e & 63;
      sKt[r * LDF + c] = sKt[r * LDF + c] * __expf(sBb[(L - 1) * LDF + c] - sBb[r * LDF + c]);
    }
    __syncthreads();
    for (int k0 = 0; k0 < KS; k0 += 16) {
      bf16x8 ah, al;
      frag_rm_f32(sKt + tr * 32 * LDF + k0, LDF, ah, al);
      const bf16x8 bh = frag_rm(sDh + tc * 32 * LDH + k0, LDH);
      const bf16x8 bl = frag_rm(sDl + tc * 32 * LDH + k0, LDH);
      mfma3(acc, ah, al, bh, bl);
    }
    __syncthreads();
  }
  const long dvo = tok0 * rsv + (long)h * a.V + v0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = tr * 32 + acc_row(i);
    if (r < L) {
      const long e = dvo + (long)r * rsv + tc * 32 + acc_col();
      if (a.dv32) a.dv32[e] = acc[i];
      if (a.dv) ((bf16*)a.dv)[e] = (bf16)acc[i];
    }
  }
}

// ===========================================================================
// gla_bwd_dqk: grid NTG * H * (K/64), XCD-mapped.  dq, dk and dG for one 64-channel slab, then the in-chunk
// suffix sums of dG (dgk before the carry of later chunks) and the chunk totals.
// ===========================================================================
template <int K>
__global__ __launch_bounds__(kThreads) void gla_bwd_dqk_kernel(const GlaArgs a) {
  // loop phase: dO, V [64][LDH] bf16 and S, dS pieces [v][c] hi/lo; post phase: q (then dG in its
  // place: each element of dG is written by the one thread that last reads that element of q), k,
  // b, dA.  Under 80 KiB, so two workgroups share a CU.
  constexpr long kLoop = 6L * 64 * LDH * 2;
  constexpr long kPost = 3L * BT * LDF * 4 + (long)BT * (BT + 1) * 4;
  __shared__ __attribute__((aligned(16))) char smem[kLoop > kPost ? kLoop : kPost];
  __shared__ float sPart[4 * KS];
  __shared__ float sTerm[KS];
  bf16* sO = (bf16*)smem;
  bf16* sV = sO + 64 * LDH;
  bf16* sSh = sV + 64 * LDH;
  bf16* sSl = sSh + 64 * LDH;
  bf16* sDh = sSl + 64 * LDH;
  bf16* sDl = sDh + 64 * LDH;
  float* sQ = (float*)smem;
  float* sK = sQ + BT * LDF;
  float* sBb = sK + BT * LDF;
  float* sG = sQ;
  float* sdA = sBb + BT * LDF;

  const int tid = threadIdx.x, w = wave_id(), l = lane_id();
  // the K / KS key blocks of a (chunk, head) unit share its operands: one XCD (L2) per unit
  int unit, kb;
  xcd_map(blockIdx.x, K / KS, a.NTG * a.H, unit, kb);
  const int gc = unit / a.H, h = unit % a.H, s0 = kb * KS;
  int n, c0, L;
  long bos;
  if (!gla_chunk(a, gc, n, c0, bos, L)) return;
  const long tok0 = bos + c0;
  const long rsk = (long)a.H * K, rsv = (long)a.H * a.V;
  const int tr = w >> 1, tc = w & 1;
  const int I = (w == 0) ? 0 : 1, J = (w == 2) ? 1 : 0;  // dA block of waves 0..2

  f32x16 dqr = zero16(), dkr = zero16(), dA = zero16();
  for (int v0 = 0; v0 < a.V; v0 += 64) {
    const long sbase = (((long)gc * a.H + h) * a.V + v0) * K + s0;
    tile_bf16(sO, (const bf16*)a.dout + tok0 * rsv + (long)h * a.V + v0, rsv, L);
    tile_bf16(sV, (const bf16*)a.v + tok0 * rsv + (long)h * a.V + v0, rsv, L);
    tile_bf16(sSh, (const bf16*)a.hT + sbase, K, 64);
    tile_bf16(sSl, (const bf16*)a.hTl + sbase, K, 64);
    tile_bf16(sDh, (const bf16*)a.dhT + sbase, K, 64);
    tile_bf16(sDl, (const bf16*)a.dhTl + sbase, K, 64);
    __syncthreads();
    for (int k0 = 0; k0 < 64; k0 += 16) {
      const bf16x8 oa = frag_rm(sO + tr * 32 * LDH + k0, LDH);
      const bf16x8 va = frag_rm(sV + tr * 32 * LDH + k0, LDH);
      dqr = mfma(oa, frag32_tr(sSh + k0 * LDH + tc * 32, LDH), dqr);
      dqr = mfma(oa, frag32_tr(sSl + k0 * LDH + tc * 32, LDH), dqr);
      dkr = mfma(va, frag32_tr(sDh + k0 * LDH + tc * 32, LDH), dkr);
      dkr = mfma(va, frag32_tr(sDl + k0 * LDH + tc * 32, LDH), dkr);
      if (w < 3) dA = mfma(frag_rm(sO + I * 32 * LDH + k0, LDH), frag_rm(sV + J * 32 * LDH + k0, LDH), dA);
    }
    __syncthreads();
  }

  // post phase
  slab_to_f32(sQ, a.q32 ? a.q32 + tok0 * rsk + (long)h * K + s0 : nullptr,
              a.q32 ? nullptr : (const bf16*)a.q16 + tok0 * rsk + (long)h * K + s0, rsk, L);
  slab_to_f32(sK, nullptr, (const bf16*)a.k + tok0 * rsk + (long)h * K + s0, rsk, L);
  slab_to_f32(sBb, a.bcum + tok0 * rsk + (long)h * K + s0, nullptr, rsk, L, true);
  if (w < 3) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int t = 32 * I + acc_row(i), s = 32 * J + acc_col();
      sdA[t * (BT + 1) + s] = (s <= t && t < L) ? a.scale * dA[i] : 0.f;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) sdA[acc_row(i) * (BT + 1) + 32 + acc_col()] = 0.f;
  }
  // final-state term of dG: rowsum over v of dS_final o S_final (last chunk of the sequence only)
  long len_seq;
  {
    long b2;
    int len2;
    seq_bounds(a.cu, n, a.T, b2, len2);
    len_seq = len2;
  }
  const bool last = (c0 + L == len_seq);
  if (last && a.ds_fin && a.s_fin_in && a.dgk) {
    const int c = tid & 63, part = tid >> 6;
    const long base = (((long)n * a.H + h) * K + s0 + c) * a.V;
    float acc_t = 0.f;
    for (int v = part; v < a.V; v += 4) acc_t += a.ds_fin[base + v] * a.s_fin_in[base + v];
    sPart[part * KS + c] = acc_t;
  }
  __syncthreads();
  if (tid < KS) {
    sTerm[tid] = (last && a.ds_fin && a.s_fin_in && a.dgk)
                     ? sPart[tid] + sPart[KS + tid] + sPart[2 * KS + tid] + sPart[3 * KS + tid]
                     : 0.f;
  }

  // intra-chunk parts.  The dq rows of block tr take the keys of block tr (the diagonal block) and,
  // for tr = 1, the keys of block 0; the dk rows (keys) of block tr take the queries of block tr and,
  // for tr = 0, the queries of block 1.  The off-diagonal block (dxo) splits its pairwise factor at
  // row mB = 32, where both factors are <= 1; the diagonal block at its middle row mR while that is
  // safe for this wave's channels (split_ok), else with one exponential per pair, in which case dqi
  // and dki carry their factors whole.
  const int mR = min(32 * tr + 16, L - 1), mB = min(32, L - 1);
  f32x16 dqi = zero16(), dki = zero16(), dxo = zero16();
  const bool fast = split_ok(sBb, LDF, 32 * tr, mR, L, tc * 32 + (l & 31));
  {
    const int c = tc * 32 + (l & 31);
    const float bm = sBb[mR * LDF + c], bb = sBb[mB * LDF + c];
    if (tr == 1) {
      for (int k0 = 0; k0 < 32; k0 += 16) {      // dq: keys of block 0
        bf16x8 ah, al, bh, bl;
        frag_rm_f32(sdA + 32 * (BT + 1) + k0, BT + 1, ah, al);
        float xb[8];
        const int kb = k0 + ((l >> 5) << 3);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int s = kb + i;
          xb[i] = sK[s * LDF + c] * __expf(bb - sBb[s * LDF + c]);
        }
        split8(xb, bh, bl);
        mfma3(dxo, ah, al, bh, bl);
      }
    } else {
      for (int k0 = 32; k0 < BT; k0 += 16) {     // dk: queries of block 1
        bf16x8 ah, al, bh, bl;
        frag_cm_f32(sdA + k0 * (BT + 1), BT + 1, ah, al);
        float xb[8];
        const int kb = k0 + ((l >> 5) << 3);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int t = kb + i;
          xb[i] = sQ[t * LDF + c] * __expf(sBb[t * LDF + c] - bb);
        }
        split8(xb, bh, bl);
        mfma3(dxo, ah, al, bh, bl);
      }
    }
    if (fast) {
      for (int k0 = 32 * tr; k0 < 32 * tr + 32; k0 += 16) {
        bf16x8 ah, al, bh, bl;
        frag_rm_f32(sdA + tr * 32 * (BT + 1) + k0, BT + 1, ah, al);
        float xb[8];
        const int kb = k0 + ((l >> 5) << 3);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int s = kb + i;
          xb[i] = sK[s * LDF + c] * __expf(bm - sBb[s * LDF + c]);
        }
        split8(xb, bh, bl);
        mfma3(dqi, ah, al, bh, bl);
      }
      for (int k0 = 32 * tr; k0 < 32 * tr + 32; k0 += 16) {
        bf16x8 ah, al, bh, bl;
        frag_cm_f32(sdA + tr * 32 + k0 * (BT + 1), BT + 1, ah, al);
        float xb[8];
        const int kb = k0 + ((l >> 5) << 3);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int t = kb + i;
          xb[i] = sQ[t * LDF + c] * __expf(sBb[t * LDF + c] - bm);
        }
        split8(xb, bh, bl);
        mfma3(dki, ah, al, bh, bl);
      }
    } else {
      // dq_r = sum_{s <= r} dA_rs k_s e^{b_r - b_s},  dk_r = sum_{t >= r} dA_tr q_t e^{b_t - b_r}
      // over the block's valid rows, one exponential (<= 1) per pair
      const int cc = tc * 32 + acc_col(), r0 = 32 * tr, r1 = min(32 * tr + 32, L);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = r0 + acc_row(i);
        float sq = 0.f, sk = 0.f;
        if (r < L) {
          const float br = sBb[r * LDF + cc];
          for (int j = r0; j <= r; ++j)
            sq += sdA[r * (BT + 1) + j] * sK[j * LDF + cc] * __expf(br - sBb[j * LDF + cc]);
          for (int j = r; j < r1; ++j)
            sk += sdA[j * (BT + 1) + r] * sQ[j * LDF + cc] * __expf(sBb[j * LDF + cc] - br);
        }
        dqi[i] = sq;
        dki[i] = sk;
      }
    }
  }
  __syncthreads();
  // combine, write dq/dk, form dG
  {
    const int c = tc * 32 + acc_col();
    const float bm = sBb[mR * LDF + c], bb = sBb[mB * LDF + c], bl_ = sBb[(L - 1) * LDF + c];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int t = tr * 32 + acc_row(i);
      const float bt = sBb[t * LDF + c];
      float dq = a.scale * __expf(bt) * dqr[i] + (fast ? __expf(bt - bm) * dqi[i] : dqi[i]);
      float dk = __expf(bl_ - bt) * dkr[i] + (fast ? __expf(bm - bt) * dki[i] : dki[i]);
      if (tr == 1) dq += __expf(bt - bb) * dxo[i];
      else dk += __expf(bb - bt) * dxo[i];
      float g = 0.f;
      if (t < L) {
        a.dq32[(tok0 + t) * rsk + (long)h * K + s0 + c] = dq;
        a.dk32[(tok0 + t) * rsk + (long)h * K + s0 + c] = dk;
        g = sQ[t * LDF + c] * dq - sK[t * LDF + c] * dk;
        if (t == L - 1) g += sTerm[c];
      }
      sG[t * LDF + c] = g;
    }
  }
  if (!a.dgk) return;
  __syncthreads();
  // suffix sums over the chunk's rows: column c = tid & 63, quarter qr = tid >> 6 (rows 16 qr ..)
  {
    const int c = tid & 63, qr = tid >> 6;
    float run = 0.f, vals[16];
#pragma unroll
    for (int j = 15; j >= 0; --j) {
      run += sG[(16 * qr + j) * LDF + c];
      vals[j] = run;
    }
    sPart[qr * KS + c] = run;
    __syncthreads();
    float off = 0.f;
    for (int p = qr + 1; p < 4; ++p) off += sPart[p * KS + c];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int t = 16 * qr + j;
      if (t < L) a.dgk[(tok0 + t) * rsk + (long)h * K + s0 + c] = vals[j] + off;
    }
    if (qr == 0) a.gk_tot[((long)gc * a.H + h) * K + s0 + c] = vals[0] + off;
  }
}

// ===========================================================================
// gla_gk_carry: grid (N*H), K threads: gk_tot[chunk] <- sum of the totals of later chunks
// (exclusive suffix over the chunks of each sequence).
// gla_gk_add: grid (NTG, H): dgk += carry of the token's chunk.
// ===========================================================================
__global__ __launch_bounds__(kThreads) void gla_gk_carry_kernel(const GlaArgs a) {
  const int unit = blockIdx.x, c = threadIdx.x;
  if (c >= a.K) return;
  const int n = unit / a.H, h = unit % a.H;
  long bos;
  int len;
  seq_bounds(a.cu, n, a.T, bos, len);
  const int nc = (len + BT - 1) / BT;
  const int gc0 = a.cu ? a.chunk_off[n] : n * a.NT;
  float acc = 0.f;
  for (int j = nc - 1; j >= 0; --j) {
    float* p = a.gk_tot + ((long)(gc0 + j) * a.H + h) * a.K + c;
    const float t = *p;
    *p = acc;
    acc += t;
  }
}

__global__ __launch_bounds__(kThreads) void gla_gk_add_kernel(const GlaArgs a) {
  const int gc = blockIdx.x, h = blockIdx.y;
  int n, c0, L;
  long bos;
  if (!gla_chunk(a, gc, n, c0, bos, L)) return;
  const long tok0 = bos + c0;
  const long rsk = (long)a.H * a.K;
  const float* carry = a.gk_tot + ((long)gc * a.H + h) * a.K;
  for (int e = threadIdx.x; e < L * a.K; e += kThreads) {
    const int t = e / a.K, c = e % a.K;
    a.dgk[(tok0 + t) * rsk + (long)h * a.K + c] += carry[c];
  }
}

// ---------------------------------------------------------------------------
// launcher
// ---------------------------------------------------------------------------
template <int K>
hipError_t launch_gla_k(int stage, const GlaArgs& a, hipStream_t st) {
  const dim3 blk(kThreads);
  const int NTG = a.NTG, H = a.H;
  switch (stage) {
    case kGlaIntra:
      hipLaunchKernelGGL(gla_intra_kernel<K>, dim3(NTG, H), blk, 0, st, a);
      break;
    case kGlaFwdState:
      hipLaunchKernelGGL(gla_state_kernel<0>, dim3(a.N * H * (K / 32) * (a.V / 32)), dim3(64), 0, st, a);
      break;
    case kGlaFwdO:
      hipLaunchKernelGGL(gla_fwd_o_kernel<K>, dim3(NTG * H * (a.V / 64)), blk, 0, st, a);
      break;
    case kGlaBwdState:
      hipLaunchKernelGGL(gla_state_kernel<1>, dim3(a.N * H * (K / 32) * (a.V / 32)), dim3(64), 0, st, a);
      break;
    case kGlaBwdDv:
      hipLaunchKernelGGL(gla_bwd_dv_kernel<K>, dim3(NTG * H * (a.V / 64)), blk, 0, st, a);
      break;
    case kGlaBwdDqk:
      hipLaunchKernelGGL(gla_bwd_dqk_kernel<K>, dim3(NTG * H * (K / KS)), blk, 0, st, a);
      break;
    case kGlaBwdGk:
      hipLaunchKernelGGL(gla_gk_carry_kernel, dim3(a.N * H), blk, 0, st, a);
      hipLaunchKernelGGL(gla_gk_add_kernel, dim3(NTG, H), blk, 0, st, a);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_gla_stage(int stage, const GlaArgs& a, hipStream_t st) {
  if (a.NTG <= 0 || a.H <= 0 || a.N <= 0) return hipSuccess;
  switch (a.K) {
    case 64: return launch_gla_k<64>(stage, a, st);
    case 128: return launch_gla_k<128>(stage, a, st);
    case 256: return launch_gla_k<256>(stage, a, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ccq
