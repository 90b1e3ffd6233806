// Argument block of the cleaning-given-z kernels (plain pointers and sizes; shared by the kernels
// and the C-ABI entry points).
#pragma once

#include <stdint.h>

namespace ccq {

struct ZCleanArgs {
  const void* q;            // bf16 [tokens, H, K]
  const void* k;            // bf16
  const void* z;            // bf16
  const float* lam;         // fp32 [tokens, H]
  const float* m0;          // fp32 [N, H, K] (nullable)
  const int64_t* cu;        // [N+1] (nullable)
  const int* chunk_idx;     // varlen: [NB, 2]
  const int* chunk_off;     // varlen: [N+1]
  float* ksum;              // [NB, H, K] block totals (forward: of k; backward: of dm)
  float* prefix;            // [NB, H, K] key sum before each block (incl. m0)    -- saved
  void* qc;                 // bf16 out
  float* m_fin;             // [N, H, K] (nullable)
  // backward
  const void* dqc16;        // bf16 upstream (or dqc32)
  const float* dqc32;
  const float* dm_fin;      // [N, H, K] (nullable)
  float* carry;             // [NB, H, K] sum of dm over later blocks (+ dm_fin)
  void* dq;                 // bf16
  void* dk;                 // bf16
  void* dz;                 // bf16
  float* dlam;              // fp32 [tokens, H] (nullable)
  float* dm0;               // fp32 [N, H, K] (nullable)
  int T, H, N, NT, NB, K, pos_off, subtract_mean;
};

}  // namespace ccq
