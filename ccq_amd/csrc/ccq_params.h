// Argument blocks of the CCQ kernels (plain pointers and sizes; shared by the
// kernels and the C-ABI entry points).
//
// Layouts (token-major, as in the reference): q, k [tokens, H, K]; v, o [tokens, H, V];
// per-token scalars [tokens, H]; tokens = B*T for dense inputs, the packed length for
// varlen inputs (B == 1 with cu_seqlens [N+1]).  States are per sequence:
// covariance [N, H, K, K], key sum [N, H, K], backbone state S [N, H, K, V].
#pragma once

#include <stdint.h>

namespace ccq {

// slices of the first pass of the column sums of partial rows (launch_sum_rows)
constexpr int kSumSlices = 32;
// partial rows of the narrow linear backward (64-row groups, at most this many)
constexpr int kNarrowBlocks = 256;

// Short causal depthwise convolution (+ activation, + per-head L2 normalisation) of the layer
// prologue: x, y, yn, dy, dyn, dx bf16 [tokens, D]; weight fp32 [D, W] (tap W-1 on the current
// token); caches fp32 [N, D, W-1] (the previous W-1 inputs of each sequence).
struct ConvArgs {
  const void* x;
  const float* w;
  const float* bias;        // [D] (nullable)
  const float* cache_in;    // (nullable = zeros)
  const int64_t* cu;        // [N+1] (nullable: N sequences of T tokens)
  void* y;                  // act(conv(x)) (nullable)
  void* yn;                 // per-head L2-normalised y (nullable)
  float* rstd;              // fp32 [tokens, D / hd] (with yn)
  float* cache_out;         // (nullable)
  const void* dy;           // bwd: gradient of y (nullable)
  const void* dyn;          // bwd: gradient of yn (nullable)
  void* dx;
  float* dw_part;           // fp32 [blocks, D * W] per-workgroup partial weight gradients
  float* db_part;           // fp32 [blocks, D] (nullable)
  long tokens;
  int T, N, D, W, hd, act;
  int tb;                   // fwd: tokens per tile (consecutive tokens one thread walks with a sliding window)
  int cg;                   // channel groups (8 channels each) per workgroup, a power of two <= 256
  int nvb;                  // virtual workgroups: a workgroup holds 256 / cg token lanes, each one of them
  float eps;
};

// Decode prologue of a CCQ-GDN layer (one token step of B sequences, T tokens each): from the rows of
// the layer's input projections (bf16, row r = b T + t, `ldx` elements apart) -- q, k, v (conv inputs)
// and a, b (decay and beta logits) -- the short convolutions + SiLU with in-place bf16 caches
// [B, D, W-1], the per-head L2 normalisation of q and k, lambda = sigmoid(lw . q_act + lb) (the
// layer's dense gate on the un-normalised activation), beta = sigmoid(b) and
// g = -exp(A_log) softplus(a + dt_bias), written to the decode step's input buffers.
struct DecProArgs {
  const void* xq;           // bf16 rows: q projection (H K), k projection (H K), v projection (H V)
  const void* xk;
  const void* xv;
  const void* xa;           // bf16 rows: a projection (H), b projection (H)
  const void* xb;
  long ldx;                 // elements between consecutive token rows
  const void* wq;           // bf16 [D, W] convolution weights (the modules' [D, 1, W])
  const void* wk;
  const void* wv;
  const void* bq;           // bf16 [D] convolution biases (nullable)
  const void* bk;
  const void* bv;
  void* cq;                 // bf16 [B, D, W-1] convolution caches, updated in place
  void* ck;
  void* cv;
  const void* lw;           // bf16 [H, H K] gate weight, [H] gate bias
  const void* lb;
  const void* alog;         // bf16 [H] A_log, dt_bias
  const void* dtb;
  void* q;                  // bf16 [B, T, H, K] normalised q, k; [B, T, H, V] v
  void* k;
  void* v;
  float* lam;               // fp32 [B, T, H]
  float* g;
  float* beta;
  int B, T, H, K, V, W, neg_eig;
  float eps;
};

// Gated RMSNorm of the layer epilogue: y = x / sqrt(mean(x^2) + eps) * w * silu(g) per row of dv
// (x, g, y, dy, dx, dg bf16 [rows, dv]; w fp32 [dv] (nullable = ones); rstd fp32 [rows]).
// Narrow linear map y = x W^T (+ b) with at most 16 outputs per row (the layers' gate projections:
// d_model -> heads, key_dim -> heads, the low-rank log gate): x [M, K] bf16 (row stride ldx), W [N, K]
// bf16, b [N] fp32 (nullable), y [M, N] bf16; backward dx [M, K] bf16 (row stride K) and per-block
// partial rows of dW [blocks, N * K] and db [blocks, N], fp32.
struct NarrowArgs {
  const void* x;
  long ldx;
  const void* w;
  const float* b;
  void* y;
  const void* dy;           // bf16 [M, N]
  void* dx;                 // bf16 [M, K] (nullable: no input gradient)
  float* dw_part;
  float* db_part;           // nullable
  long M;
  int K;
  int N;
  int rpb;                  // rows per block (backward)
};

struct GNormArgs {
  const void* x;
  const void* g;
  const float* w;
  void* y;
  float* rstd;
  const void* dy;
  void* dx;
  void* dg;
  float* dw_part;           // fp32 [blocks, dv] (nullable)
  long rows;
  int dv;
  int lr;                   // lanes per row: the next power of two of dv / 8 (64 / lr rows per wavefront)
  float eps;
  long ldg;                 // forward: gate row r at g + (r / gper) * ldg + (r % gper) * dv
  int gper;                 //   (contiguous rows: gper = 1, ldg = dv)
};

struct L2NormArgs {
  const void* x;            // bf16 [rows, D]
  void* y;                  // bf16 [rows, D]
  float* rstd;              // fp32 [rows]
  const float* dy32;        // bwd: fp32 upstream (or dy16)
  const void* dy16;
  void* dx;                 // bf16 [rows, D]
  long rows;
  int D;
  int lr;                   // vector kernels: lanes per row (next power of two of D / 8), 64 / lr rows per wave
  float eps;
};

}  // namespace ccq

namespace ccq {

// Gated delta rule (chunk size 64).  Internal buffers (all caller-allocated):
//   gcum [tokens, H] fp32         in-chunk cumulative log decay
//   tmat [NTG, H, 64, 64] fp32    T = (I + A)^-1 of the WY representation
//   w, wl [tokens, H, K] bf16     w = T diag(beta exp(G)) K as a hi/lo pair
//   u    [tokens, H, V] fp32      u = T diag(beta) V
//   hT   [NTG, H, V, K] 16-bit    state at each chunk start (transposed): int16 rows with hTl
//                                 [NTG, H, V] fp32 their power-of-two scales (snap16), else bf16
//                                 with hTl [NTG, H, V, K] bf16 its low part
//   U    [tokens, H, V] fp32      U = u - w S (pseudo-values after the delta correction)
//   PT   [NTG, H, 64, 64] fp32    P^T, P = scale (Qc K^T o Gamma), causal incl. diagonal
//   dU   [tokens, H, V] fp32      gradient of U
//   dhT  [NTG, H, V, K] 16-bit    gradient of the state after each chunk (transposed), dhTl as hTl
//   dq32 / dkp32 / dw32 [tokens, H, K] fp32, dgp [K/64, tokens, H] fp32; for K = V = 128 dkp32 and
//                                 dw32 hold int16 [tokens, H, K] with fp32 power-of-two scales
//                                 dkp_sc / dw_sc [tokens, H, K/32] (one per row and 32-column block)
enum GdnStage { kGdnPrep = 0, kGdnFwdState, kGdnFwdO, kGdnBwdState, kGdnBwdDqkw, kGdnBwdWy };

struct GdnArgs {
  const void* qc16;         // bf16 cleaned query (or qc32)
  const float* qc32;        // fp32 cleaned query
  const void* k;            // bf16 [tokens, H, K]
  const void* v;            // bf16 [tokens, H, V]
  const float* g;           // fp32 [tokens, H] log decay (nullable: no decay)
  const float* beta;        // fp32 [tokens, H]
  const float* s0;          // fp32 [N, H, K, V] initial state (nullable)
  const int64_t* cu;        // [N+1] (nullable)
  const int* chunk_idx;     // [NTG, 2] (sequence, chunk) for varlen
  const int* chunk_off;     // [N+1] first global chunk of each sequence (varlen)
  float* gcum;
  float* tmat;
  void* w;
  void* wl;                 // bf16 low part of w (w + wl ~ fp32)
  float* u;
  void* hT;
  void* hTl;                // row scales of hT (snap16), else its bf16 low parts
  float* U;
  float* PT;
  void* o;                  // bf16 [tokens, H, V]
  float* s_fin;             // fp32 [N, H, K, V] (nullable)
  // backward
  const void* dout;         // bf16 [tokens, H, V]
  const float* ds_fin;      // fp32 [N, H, K, V] (nullable)
  float* dU;
  void* dhT;
  void* dhTl;               // row scales of dhT (snap16), else its bf16 low parts
  float* dq32;              // gradient of the cleaned query
  float* dkp32;             // gradient of k (state/output part)
  float* dw32;
  float* dkp_sc;            // scales of dkp32 / dw32 in their int16 form (nullable: fp32)
  float* dw_sc;
  float* dgp;
  float* dk32;              // gradient of k (total GDN part)
  void* dv;                 // bf16 [tokens, H, V]
  float* dbeta;             // fp32 [tokens, H]
  float* dg;                // fp32 [tokens, H]
  float* ds0;               // fp32 [N, H, K, V] (nullable)
  float scale;
  int T, H, N, NT, NTG;     // NT: chunks per sequence (dense); NTG: total chunks
  // state and state-gradient snapshots as int16 rows with a power-of-two scale per row (hT / dhT hold
  // the integers, hTl / dhTl the fp32 row scales [NTG * H, V]) instead of hi/lo bf16 pairs: set for
  // K = 64 and 256 and for K = V = 128, whose dq/dk/dw (and K = 256 output) kernels read that form
  int snap16;
};

}  // namespace ccq

namespace ccq {

// Gated linear attention (chunk size 64, per-channel log decay gk).  Buffers (caller-allocated):
//   bcum [tokens, H, K] fp32      in-chunk cumulative log decay b_t = sum_{s<=t in chunk} gk_s
//   A    [NTG, H, 64, 64] fp32    scale * sum_c q_tc k_sc exp(b_tc - b_sc), causal incl. diagonal
//   hT   [NTG, H, V, K] bf16      state at each chunk start (transposed), hTl its low part
//   dhT  [NTG, H, V, K] bf16      gradient of the state after each chunk (transposed), dhTl low part
//   gk_tot [NTG, H, K] fp32       per-chunk totals of d(cumulative decay), then their suffix carry
enum GlaStage { kGlaIntra = 0, kGlaFwdState, kGlaFwdO, kGlaBwdState, kGlaBwdDv, kGlaBwdDqk, kGlaBwdGk };

struct GlaArgs {
  const void* q16;          // bf16 query (or q32)
  const float* q32;         // fp32 query (the cleaned query)
  const void* k;            // bf16 [tokens, H, K]
  const void* v;            // bf16 [tokens, H, V]
  const float* gk;          // fp32 [tokens, H, K] per-channel log decay (nullable: no decay)
  const float* h0;          // fp32 [N, H, K, V] (nullable)
  const int64_t* cu;        // [N+1] (nullable)
  const int* chunk_idx;     // varlen: [NTG, 2] (sequence, chunk)
  const int* chunk_off;     // varlen: [N+1]
  float* bcum;
  float* A;
  void* hT;
  void* hTl;
  void* o;                  // bf16 [tokens, H, V]
  float* s_fin;             // fp32 [N, H, K, V] (nullable)
  // backward
  const void* dout;         // bf16 [tokens, H, V]
  const float* ds_fin;      // fp32 [N, H, K, V] (nullable)
  const float* s_fin_in;    // fp32 [N, H, K, V] forward final state (nullable; needed with ds_fin for dgk)
  void* dhT;
  void* dhTl;
  float* dq32;              // fp32 [tokens, H, K]
  float* dk32;              // fp32 [tokens, H, K]
  void* dv;                 // bf16 [tokens, H, V] (nullable when dv32 is set)
  float* dv32;              // fp32 [tokens, H, V] (nullable)
  float* dgk;               // fp32 [tokens, H, K] (nullable)
  float* gk_tot;
  float* dh0;               // fp32 [N, H, K, V] (nullable)
  float scale;
  int T, H, N, NT, NTG, K, V;
};

}  // namespace ccq
