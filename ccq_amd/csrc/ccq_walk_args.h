// Argument block of the column-walk cleaning kernels (plain pointers and sizes; shared by the
// kernels and the C-ABI entry points).
//
// Layouts (token-major, as in the reference): q, k [tokens, H, K] bf16; per-token scalars
// [tokens, H]; states per sequence: covariance [N, H, K, K], key sum [N, H, K] (fp32).
#pragma once

#include <stdint.h>

namespace ccq {

// Tokens per chunk of the walks: 64, or 32 for K = 256 (the full-width tiles of the backward
// walks must fit in LDS).
constexpr int walk_chunk(int K) { return K > 128 ? 32 : 64; }

struct WalkArgs {
  const void* q;            // bf16 [tokens, H, K]
  const void* k;            // bf16 [tokens, H, K]
  const float* lam;         // fp32 [tokens, H] (forward; unused with the fused gate)
  const float* gate_w;      // fp32 [H, K] (nullable: lambda is given)
  const float* gate_b;      // fp32 [H]
  float* lam_out;           // fp32 [tokens, H] gate output (nullable)
  const float* h0;          // fp32 [N, H, K, K] (nullable)
  const float* m0;          // fp32 [N, H, K] (nullable)
  const int64_t* cu;        // [N+1] (nullable)
  const int* chunk_idx;     // varlen: [NTG, 2] (sequence, chunk) of walk chunks, -1 for padding
  const int* chunk_off;     // varlen: [N+1] first global chunk of each sequence
  // forward -> backward
  float* z;                 // fp32 [tokens, H, K] covariance read z_t = C_t^T q_t
  float* srow;              // fp32 [tokens, H] s_t = m_t . q_t
  float* mpre;              // fp32 [NTG, H, K] key sum before each chunk (incl. m0)
  // forward outputs
  void* qc;                 // bf16 [tokens, H, K] (nullable)
  float* qc32;              // fp32 [tokens, H, K] (nullable)
  float* h_fin;             // fp32 [N, H, K, K] (nullable)
  float* m_fin;             // fp32 [N, H, K] (nullable)
  // backward
  const float* dqc32;       // fp32 upstream gradient (or dqc16)
  const void* dqc16;        // bf16 upstream gradient
  const float* lam_used;    // fp32 [tokens, H] lambda of the forward (given or gate output)
  const float* dk_extra;    // fp32 [tokens, H, K] added into dk (nullable)
  const float* dh_fin;      // fp32 [N, H, K, K] (nullable)
  const float* dm_fin;      // fp32 [N, H, K] (nullable)
  float* sc;                // fp32 [tokens, H, 4]: -lambda_t/pos_t, ds_t, dlambda_t (or dlogit_t), -s_t/pos_t
  void* dq;                 // bf16 (nullable)
  float* dq32;              // fp32 (nullable)
  void* dk;                 // bf16 (nullable)
  float* dk32;              // fp32 (nullable)
  float* dlam;              // fp32 [tokens, H] (nullable)
  float* dw_part;           // fp32 [NTG, H, K] gate partials
  float* db_part;           // fp32 [NTG, H]
  float* dmsum;             // fp32 [NTG, H, K] per-chunk column sums of dm (subtract_mean)
  void* dzh;                // bf16 [tokens, H, K] dz_t = F_t dqc_t, hi (nullable: the walks form dz)
  void* dzl;                // bf16 [tokens, H, K] low part
  float* dh0;               // fp32 [N, H, K, K] (nullable)
  float* dm0;               // fp32 [N, H, K] (nullable)
  // segment walks (K in {64, 128}): per (sequence, head, segment) totals
  float* segD;              // saved: fp32 [N*H, nseg, K, K] sum of k k^T over the segment
  float* segM;              // saved: fp32 [N*H, nseg, K] sum of k over the segment
  float* segG;              // workspace: fp32 [N*H, nseg, K, K] sum of q dz^T over the segment
  float* segDM;             // workspace: fp32 [N*H, nseg, K] sum of dm over the segment
  int T, H, N, NT, NTG, K, pos_off, subtract_mean;
  int nseg;                 // time segments per sequence of the segment walks
};

// stages of launch_cwalk
enum WalkStage { kWalkFwd = 0, kWalkRows, kWalkDq, kWalkDk };
// stages of launch_cseg (segment walks, K in {64, 128})
enum SegStage { kSegSum = 0, kSegFwd, kSegDq, kSegGsum, kSegDk };

}  // namespace ccq
