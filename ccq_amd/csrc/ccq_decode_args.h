// Argument block of the recurrent (decode) step kernels (plain pointers and sizes; shared by the
// kernels and the C-ABI entry points).
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace ccq {

// Size of the per-device scratch array of ccq_gdn_decode_noalloc (the decode workspace: the fp32
// cleaned query and key of the call's tokens, 8 bytes per token, head and key channel).
constexpr size_t kDecodeScratchBytes = (size_t)8 << 20;
constexpr int kMaxDevices = 64;
constexpr int kDecodeLayerMaxQ = 2048;  // H K of the layer form

// The layer form (ccq_gdn_layer_decode_step): q and k read from the layer's projection rows, after
// the short convolutions and SiLU that the projection kernel's epilogue applied, and L2-normalised
// here; lambda = sigmoid(lambda gate of the whole q activation).
struct DecodeLayer {
  const void* x;           // bf16 rows [B T, ldx]: q (H K) at column oq, k (H K) at ok
  long ldx;
  int oq, ok;
  const void* lw;          // bf16 [H, H K] lambda gate weight, [H] bias (nullable)
  const void* lb;
  float l2eps;
};

struct DecodeArgs {
  const void* q;           // bf16 [tokens, H, K]
  const void* k;           // bf16 [tokens, H, K]
  const void* v;           // bf16 [tokens, H, V]
  const float* lam;        // fp32 [tokens, H] (or gate_w / gate_b)
  const float* gate_w;     // fp32 [H, K] (nullable)
  const float* gate_b;     // fp32 [H]
  const float* g;          // GDN: fp32 [tokens, H] log decay (nullable)
  const float* beta;       // GDN: fp32 [tokens, H]
  const float* gk;         // GLA: fp32 [tokens, H, K] log decay of the key rows (nullable)
  const float* gv;         // GLA: fp32 [tokens, H, V] log decay of the value columns (nullable)
  const float* S_in;       // [N, H, K, V] (nullable = 0)
  const float* C_in;       // [N, H, K, K] (nullable = 0)
  const float* m_in;       // [N, H, K] (nullable = 0)
  float* S_out;            // nullable
  float* C_out;            // nullable
  float* m_out;            // nullable
  void* o;                 // bf16 [tokens, H, V]
  float* qc;               // workspace fp32 [tokens, H, K]: cleaned query
  float* kn;               // workspace fp32 [tokens, H, K]: (normalised) key
  const int64_t* cu;       // [N+1] (nullable)
  const int* pos_dev;      // device int: the position offset (nullable: pos_off)
  // in-place step (nullable): after the clean kernel, m_dst[0, m_count) = m_src and *pos_adv += T
  float* m_dst;
  const float* m_src;
  long m_count;
  int* pos_adv;
  float scale;
  int T, H, N, K, V, pos_off, subtract_mean, l2norm, ccq, gla;
  int reverse;             // GLA: the backbone recurrence runs from the last token to the first
  long vld;                // elements between the v rows of consecutive tokens (0: H V)
  DecodeLayer lay;         // the layer form (lay.x set)
};

}  // namespace ccq
