// Recurrent (decode) step of CCQ-GDN and CCQ-GLA on gfx950: a few tokens per sequence against the
// cached states (S [K, V], C [K, K], m [K], fp32), as the reference's fused_recurrent_ccq_gdn /
// fused_recurrent_ccq_gla compute it (ccq/ops/ccq_gdn/fused_recurrent.py:18-75 with
// fused_clean.py:34-83; ccq/ops/ccq_gla/fused_recurrent.py:9-51).  Per token t of a sequence:
//   q, k <- l2norm(q), l2norm(k)   (optional, outputs rounded to bf16 as fla's l2norm returns them)
//   C <- C + k k^T;  m <- m + k;  z = C^T q;  s = m . q;  pos = max(t + 1 + position_offset, 1)
//   q_clean = q - lambda (z / pos - s m / pos^2)          (mean term only with subtract_mean)
//   GDN: S <- e^g diag(e^gk) S diag(e^gv) (gk, gv optional);  u = beta (v - S^T k);  S <- S + k u^T;
//        o = S^T (scale q_clean)
//   GLA: S <- diag(e^gk) S diag(e^gv) + k v^T;  o = S^T (scale q_clean)  (optionally from the last
//        token to the first: `reverse`, the cleaning itself always runs forwards)
//
// The step is HBM-bound (each state element is read and written once per call).  Two launches:
//   decode_clean   grid (N*H, K/32): each workgroup owns 32 columns of C (held in registers across
//                  the call's tokens) and writes the fp32 cleaned query of those columns;
//   decode_backbone grid (N*H, V/32): each workgroup owns 32 columns of S, reads the cleaned query;
//                  an in-place step (device-held position) also moves the new key sum over the
//                  cached one and advances the position here.
// Thread (columns 4 (tid % 8) .. + 3 of the block, row group tid / 8) holds K/32 consecutive rows of them.
#include <mutex>

#include "ccq_tile.h"
#include "ccq_decode_args.h"

namespace ccq {

namespace {

// (every thread of the workgroup calls it)
__device__ __forceinline__ float block_sum256(float x, float* red) {
  x = wave_total(x);
  if (lane_id() == 0) red[wave_id()] = x;
  __syncthreads();
  const float s = red[0] + red[1] + red[2] + red[3];
  __syncthreads();
  return s;
}

}  // namespace

// Column blocks: a workgroup owns DC = 32 columns of a state and all of its rows.  A thread holds
// four consecutive columns (one 16-byte piece) of RPT = K / RG consecutive rows, RG = 32 row groups:
// every state load or store of a wave covers eight whole 128-byte row pieces, so a 32-column slice
// moves in K / 32 wide instructions per thread (one 4-byte access per instruction moved only a
// quarter of that per issue slot).  Column sums over the rows go through LDS in two levels.
constexpr int DC = 32, NQ = DC / 4, RG = kThreads / NQ;

// A thread's RPT rows x 4 columns of a state slice to HBM (row stride ld).
template <int K>
__device__ __forceinline__ void store_cols(float* base, int ld, int rg, int c4, const f32x4 (&x)[K / RG]) {
#pragma unroll
  for (int r = 0; r < K / RG; ++r) *(f32x4*)(base + (long)(rg * (K / RG) + r) * ld + c4) = x[r];
}

// Sums of three values over the workgroup with one barrier (each wave's totals, then the four waves'
// in order); every thread calls it, and consecutive uses of `red` are a barrier apart.
__device__ __forceinline__ void block_sum3(float& x, float& y, float& z, float (*red)[4]) {
  x = wave_total(x);
  y = wave_total(y);
  z = wave_total(z);
  if (lane_id() == 0) {
    red[0][wave_id()] = x;
    red[1][wave_id()] = y;
    red[2][wave_id()] = z;
  }
  __syncthreads();
  x = red[0][0] + red[0][1] + red[0][2] + red[0][3];
  y = red[1][0] + red[1][1] + red[1][2] + red[1][3];
  z = red[2][0] + red[2][1] + red[2][2] + red[2][3];
}

// LAYER: q and k from the layer's projection rows (after the short convolutions), L2-normalised per
// head here, and lambda from the whole q activation (ccq/gdn/layer.py:288-316).
// Per token: one barrier for the three sums of the front (|q|^2, |k|^2, the lambda logit), one after
// the normalised q and k reach LDS, one for the column sums of z, which carry s = m . q along; the
// running key sum stays in registers (row tid for s, column j0 + tid for the correction).
template <int K, bool LAYER>
__global__ __launch_bounds__(kThreads) void decode_clean_kernel(const DecodeArgs a) {
  constexpr int RPT = K / RG;  // rows per thread
  static_assert(RPT >= 1, "K >= 32");
  __shared__ __attribute__((aligned(16))) float sq[K], sk[K];
  __shared__ __attribute__((aligned(16))) float mid[4][DC + 4];  // per wave: z column sums, then s
  __shared__ float red[3][4], red2[4];
  const int tid = threadIdx.x, cq = tid % NQ, rg = tid / NQ;
  const int unit = blockIdx.x, n = unit / a.H, h = unit % a.H;
  const int j0 = blockIdx.y * DC, j4 = j0 + 4 * cq;
  long bos;
  int len;
  seq_bounds(a.cu, n, a.T, bos, len);
  const int pos_off = a.pos_dev ? *a.pos_dev : a.pos_off;

  // layer form: a token's q / k values and the lambda gate's operands from the projection rows, as
  // bf16 bit patterns (converting them at the load would wait for them there); every load
  // unconditional, from a clamped address, masked after (a load under a branch is waited for at the
  // branch's end).  The gate's q row and weight row come as one 16-byte piece of 8 channels per thread.
  constexpr int QV = kDecodeLayerMaxQ / kThreads;
  static_assert(QV == 8, "one 16-byte piece of the q row per thread");
  struct Rows {
    u32x4 q, lw;
    unsigned yq, yk, lb;
  };
  auto u16 = [](const bf16* p) { return (unsigned)*(const unsigned short*)p; };
  auto f16 = [](unsigned b) { return __uint_as_float(b << 16); };
  auto layer_load = [&](long tok) {
    const DecodeLayer& L = a.lay;
    const bf16* xr = (const bf16*)L.x + tok * L.ldx;
    const int D = a.H * K, c8 = min(QV * tid, D - QV), ck = min(tid, K - 1);
    Rows r;
    r.q = *(const u32x4*)(xr + L.oq + c8);
    r.lw = *(const u32x4*)((const bf16*)L.lw + (long)h * D + c8);
    r.yq = u16(xr + L.oq + h * K + ck);
    r.yk = u16(xr + L.ok + h * K + ck);
    r.lb = u16((const bf16*)(L.lb ? L.lb : L.lw) + (L.lb ? h : 0));
    return r;
  };
  Rows first{};
  if constexpr (LAYER) first = layer_load(bos);
  // (the rows' and the key sum's loads go out ahead of the slice's: the compiler would otherwise
  // issue the slice's first, whose addresses are ready earlier)
  __builtin_amdgcn_sched_barrier(0);
  // the cached key sum of row tid and of column j0 + tid through a buffer resource of no records when
  // there is none (loads past the records return zeros: no branch)
  float m_row, m_col;
  {
    const auto rm = buf_rsrc(a.m_in ? a.m_in + (long)unit * K : nullptr, a.m_in ? K * 4 : 0);
    m_row = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rm, tid * 4, 0, 0));
    m_col = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rm, (j0 + (tid & (DC - 1))) * 4, 0, 0));
  }
  __builtin_amdgcn_sched_barrier(0);
  // the covariance slice, issued after the rows and the key sum (a wait for those does not wait for
  // the slice), through a buffer resource of no records when there is no state
  f32x4 creg[RPT];
  {
    const auto rc = buf_rsrc(a.C_in ? a.C_in + (long)unit * K * K : nullptr, a.C_in ? K * K * 4 : 0);
#pragma unroll
    for (int r = 0; r < RPT; ++r)
      creg[r] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rc, ((rg * RPT + r) * K + j4) * 4, 0, 0));
  }

  const bool norm = LAYER || a.l2norm;
  // token t of the sequence (layer form: its rows r)
  auto token = [&](int t, const Rows& r) {
    const long tok = bos + t;
    float yq, yk, part = 0.f, lb = 0.f;
    if constexpr (LAYER) {
      yq = tid < K ? f16(r.yq) : 0.f;
      yk = tid < K ? f16(r.yk) : 0.f;
      if (QV * tid < a.H * K) {
#pragma unroll
        for (int e = 0; e < QV / 2; ++e) {
          part += __uint_as_float(r.lw[e] << 16) * __uint_as_float(r.q[e] << 16);
          part += __uint_as_float(r.lw[e] & 0xffff0000u) * __uint_as_float(r.q[e] & 0xffff0000u);
        }
      }
      lb = a.lay.lb ? f16(r.lb) : 0.f;
    } else {
      const bf16* qg = (const bf16*)a.q + (tok * a.H + h) * K;
      const bf16* kg = (const bf16*)a.k + (tok * a.H + h) * K;
      yq = tid < K ? (float)qg[tid] : 0.f;
      yk = tid < K ? (float)kg[tid] : 0.f;
    }
    float ssq = yq * yq, ssk = yk * yk;
    if (norm) block_sum3(ssq, ssk, part, red);
    const float eps = LAYER ? a.lay.l2eps : 1e-6f;
    const float qv = norm ? (float)(bf16)(yq * rsqrtf(ssq + eps)) : yq;
    const float kv = norm ? (float)(bf16)(yk * rsqrtf(ssk + eps)) : yk;
    if (tid < K) {
      sq[tid] = qv;
      sk[tid] = kv;
    }
    if (blockIdx.y == 0 && tid < K) a.kn[(tok * a.H + h) * K + tid] = kv;
    if (!a.ccq) {
      if (blockIdx.y == 0 && tid < K) a.qc[(tok * a.H + h) * K + tid] = qv;
      __syncthreads();
      return;
    }
    // lambda
    float lam;
    if constexpr (LAYER) {
      lam = (float)(bf16)(1.f / (1.f + expf(-(float)(bf16)(part + lb))));
    } else if (a.gate_w) {
      const float x = tid < K ? a.gate_w[(long)h * K + tid] * qv : 0.f;
      lam = sigmoidf_(block_sum256(x, red2) + a.gate_b[h]);
    } else {
      lam = a.lam[tok * a.H + h];
    }
    // running key sum; this thread's term of s = m . q
    m_row += kv;
    const float sp = m_row * qv;
    __syncthreads();
    m_col += sk[j0 + (tid & (DC - 1))];
    // C column update and partial z over this thread's rows
    const f32x4 kj = *(const f32x4*)(sk + j4);
    f32x4 zp = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
      const int i = rg * RPT + r;
      creg[r] += sk[i] * kj;
      zp += creg[r] * sq[i];
    }
    // the final state leaves as soon as it is formed (its stores overlap the reduction below)
    if (t == len - 1 && a.C_out) store_cols<K>(a.C_out + (long)unit * K * K, K, rg, j4, creg);
    // column sums of z within each wave (its eight row groups: DPP, then two lane swaps) and the
    // wave's total of s, to LDS; after one barrier thread tid < DC adds the four waves' parts
    {
      f32x4 y;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float v = zp[c] + dppf<0x128>(zp[c]);  // row_ror:8 (lane l ^ 8 of the 16-lane row)
        v += __shfl_xor(v, 16);
        v += __shfl_xor(v, 32);
        y[c] = v;
      }
      const float sw = wave_total(sp);
      const int l = lane_id();
      if (l < NQ) *(f32x4*)&mid[wave_id()][4 * l] = y;
      if (l == 0) mid[wave_id()][DC] = sw;
    }
    __syncthreads();
    if (tid < DC) {
      const float z = (mid[0][tid] + mid[1][tid]) + (mid[2][tid] + mid[3][tid]);
      const float s = (mid[0][DC] + mid[1][DC]) + (mid[2][DC] + mid[3][DC]);
      float pos = (float)(t + 1 + pos_off);
      pos = pos < 1.f ? 1.f : pos;
      float corr = z / pos;
      if (a.subtract_mean) corr -= s * m_col / (pos * pos);
      a.qc[(tok * a.H + h) * K + j0 + tid] = sq[j0 + tid] - lam * corr;
    }
    // (without the front's barrier the next token's q and k would overwrite what this one reads)
    if (!norm) __syncthreads();
  };
  // the first token apart from the others: a path shared with their row loads would wait for those
  // at its join, which on the first token's path covers the slice's loads
  if (len > 0) token(0, first);
  for (int t = 1; t < len; ++t) {
    Rows r{};
    if constexpr (LAYER) r = layer_load(bos + t);
    token(t, r);
  }
  // (no token, or the plain step without cleaning: the state as it came in)
  if (a.C_out && (len == 0 || !a.ccq)) store_cols<K>(a.C_out + (long)unit * K * K, K, rg, j4, creg);
  if (a.m_out && tid < DC) a.m_out[(long)unit * K + j0 + tid] = m_col;
}

// One token's operands, as loaded: the cleaned query, the key and the key decay's exponent of row
// tid, this thread's four value columns (bf16 bits) and their decay exponents, the token's g and
// beta.  Optional inputs come through buffer resources of no records (zeros: e^0 = 1 exactly).
struct BbOps {
  float q, k, gk, g, beta;
  u32x2 v;
  f32x4 gv;
};

// Per token: the decayed state's column sums against k and the output's against the cleaned query,
// each in one LDS exchange with one barrier (every thread adds the four waves' parts of the columns
// it needs).  The token's operands are loaded ahead of the state slice, and the new key sum's copy
// over the cached one runs last: a load issued after the slice is waited for with the slice.
template <int K>
__global__ __launch_bounds__(kThreads) void decode_backbone_kernel(const DecodeArgs a) {
  constexpr int RPT = K / RG;
  static_assert(RPT >= 1, "K >= 32");
  __shared__ __attribute__((aligned(16))) float sq[K], sk[K], sgk[K];
  __shared__ __attribute__((aligned(16))) float mp[4][DC], mo[4][DC];
  const int tid = threadIdx.x, cq = tid % NQ, rg = tid / NQ;
  const int unit = blockIdx.x, n = unit / a.H, h = unit % a.H;
  const int V = a.V, v0 = blockIdx.y * DC, v4 = v0 + 4 * cq;
  long bos;
  int len;
  seq_bounds(a.cu, n, a.T, bos, len);

  // (every load through a buffer resource, of no records for an absent input or when `on` is false:
  // no branch, whose join would make the waits after it cover the state slice's loads)
  auto bb_load = [&](long tok, bool on) {
    BbOps o;
    const long row = tok * a.H + h;
    auto ld1 = [&](const float* p, int bytes, int off) {
      return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(buf_rsrc(on ? p : nullptr, on && p ? bytes : 0), off, 0, 0));
    };
    o.q = ld1(a.qc + row * K, K * 4, tid * 4);
    o.k = ld1(a.kn + row * K, K * 4, tid * 4);
    o.gk = ld1(a.gk ? a.gk + row * K : nullptr, K * 4, tid * 4);
    o.g = ld1(a.g ? a.g + row : nullptr, 4, 0);
    o.beta = ld1(a.beta ? a.beta + row : nullptr, 4, 0);
    const bf16* vr = (const bf16*)a.v + (a.vld ? tok * a.vld + (long)h * V : row * V);
    o.v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(buf_rsrc(on ? vr : nullptr, on ? V * 2 : 0), v4 * 2, 0, 0));
    o.gv = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                         buf_rsrc(on && a.gv ? a.gv + row * V : nullptr, on && a.gv ? V * 4 : 0), v4 * 4, 0, 0));
    return o;
  };
  // (the cleaned queries of every token are ready: the backbone may run backwards in time)
  auto tok_of = [&](int tt) { return bos + (a.reverse ? len - 1 - tt : tt); };
  // the slice's byte offset of this thread's first row, formed before the operand loads (address
  // arithmetic placed after them can land on a register a pending load writes and wait for it);
  // row r adds r V 4 bytes as the scalar offset
  int soff = (rg * RPT * V + v4) * 4;
  asm volatile("" : "+v"(soff));
  const BbOps first = bb_load(tok_of(0), len > 0);
  __builtin_amdgcn_sched_barrier(0);
  f32x4 sreg[RPT];
  {
    const auto rs = buf_rsrc(a.S_in ? a.S_in + (long)unit * K * V : nullptr, a.S_in ? K * V * 4 : 0);
#pragma unroll
    for (int r = 0; r < RPT; ++r)
      sreg[r] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, soff, r * V * 4, 0));
  }

  // the column sums of x over the RG row groups: within each wave (its eight row groups: DPP, then
  // two lane swaps) to mid, then (after the caller's barrier) the four waves' parts
  auto colpart = [&](float (*mid)[DC], const f32x4& x) {
    f32x4 y;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float v = x[c] + dppf<0x128>(x[c]);  // row_ror:8 (lane l ^ 8 of the 16-lane row)
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      y[c] = v;
    }
    if (lane_id() < NQ) *(f32x4*)&mid[wave_id()][4 * lane_id()] = y;
  };
  auto token = [&](int tt, const BbOps& op) {
    const long tok = tok_of(tt);
    if (tid < K) {
      sq[tid] = op.q;
      sk[tid] = op.k;
      sgk[tid] = __expf(op.gk);
    }
    __syncthreads();
    f32x4 vt, dv;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const unsigned w = op.v[c >> 1];
      vt[c] = __uint_as_float((c & 1) ? (w & 0xffff0000u) : (w << 16));
      dv[c] = __expf(op.gv[c]);
    }
    if (a.gla) {
#pragma unroll
      for (int r = 0; r < RPT; ++r) {
        const int i = rg * RPT + r;
        sreg[r] = sgk[i] * sreg[r] * dv + sk[i] * vt;
      }
    } else {
      const f32x4 dec = __expf(op.g) * dv;
      f32x4 p = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < RPT; ++r) {
        sreg[r] *= dec * sgk[rg * RPT + r];
        p += sreg[r] * sk[rg * RPT + r];
      }
      colpart(mp, p);
      __syncthreads();
      const f32x4 ks = (*(const f32x4*)&mp[0][4 * cq] + *(const f32x4*)&mp[1][4 * cq]) +
                       (*(const f32x4*)&mp[2][4 * cq] + *(const f32x4*)&mp[3][4 * cq]);
      const f32x4 u = op.beta * (vt - ks);
#pragma unroll
      for (int r = 0; r < RPT; ++r) sreg[r] += sk[rg * RPT + r] * u;
    }
    if (tt == len - 1 && a.S_out) store_cols<K>(a.S_out + (long)unit * K * V, V, rg, v4, sreg);
    f32x4 po = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < RPT; ++r) po += sreg[r] * sq[rg * RPT + r];
    colpart(mo, po);
    __syncthreads();
    if (tid < DC) {
      const float x = (mo[0][tid] + mo[1][tid]) + (mo[2][tid] + mo[3][tid]);
      ((bf16*)a.o)[(tok * a.H + h) * V + v0 + tid] = (bf16)(a.scale * x);
    }
  };
  // the first token apart from the others (a path shared with their operand loads would wait for
  // those at its join, which on the first token's path covers the slice's loads)
  if (len > 0) token(0, first);
  for (int tt = 1; tt < len; ++tt) token(tt, bb_load(tok_of(tt), true));
  if (a.S_out && len == 0) store_cols<K>(a.S_out + (long)unit * K * V, V, rg, v4, sreg);

  // end of an in-place step (the clean kernel, launched before in the same stream, has read the
  // cached key sum and the position): the new key sum replaces the cached one, the position
  // advances by the step's tokens
  if (a.m_dst) {
    const long nthreads = (long)gridDim.x * gridDim.y * kThreads;
    const long gid = ((long)blockIdx.y * gridDim.x + blockIdx.x) * kThreads + tid;
    for (long i = gid; i < a.m_count; i += nthreads) a.m_dst[i] = a.m_src[i];
  }
  if (a.pos_adv && blockIdx.x == 0 && blockIdx.y == 0 && tid == 0) *a.pos_adv += a.T;
}

template <int K>
hipError_t launch_decode_k(const DecodeArgs& a, hipStream_t st) {
  const int units = a.N * a.H;
  if (a.lay.x)
    hipLaunchKernelGGL((decode_clean_kernel<K, true>), dim3(units, K / DC), dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((decode_clean_kernel<K, false>), dim3(units, K / DC), dim3(kThreads), 0, st, a);
  hipLaunchKernelGGL(decode_backbone_kernel<K>, dim3(units, a.V / DC), dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

// Scratch of the decode entry point that allocates nothing (ccq_gdn_decode_noalloc): a file-scope
// device array, one copy per GPU, held until the process ends.  Its device address is looked up
// once per device (with that device current) and kept; host code never passes the array's name
// itself to a kernel.
static __device__ __align__(256) char scratch[kDecodeScratchBytes];

hipError_t decode_scratch(hipStream_t st, void** out) {
  static std::mutex mu;
  static void* ptrs[kMaxDevices] = {};
  int cur = 0, dev = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return e;
  dev = cur;
  if (st != nullptr && (e = hipStreamGetDevice(st, &dev)) != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> g(mu);
  if (ptrs[dev] == nullptr) {
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) return e;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) {
      const hipError_t r = hipSetDevice(cur);
      if (e == hipSuccess) e = r;
    }
    if (e != hipSuccess) return e;
    ptrs[dev] = p;
  }
  *out = ptrs[dev];
  return hipSuccess;
}

// ===========================================================================
// Decode linear map: y[m][n] = sum_k x[m][k] W[n][k] (+ r[m][n]) for M <= 16 token rows (a decode
// step's projections: the weight is read once and dominates the bytes).  Workgroup: 16 output
// columns, 16 waves splitting the contraction into interleaved 32-wide steps (at most 8 per wave, so
// four waves per SIMD keep a whole workgroup's loads in flight at once); per step a 16x16x32 MFMA
// with the weight's 16 rows as the A operand (16 bytes per lane, straight from HBM, every step of
// the wave in flight at once) and the token rows as the B operand (L2-resident).  The waves' partial
// 16x16 tiles meet in LDS; the result (lane (m, n / 4): four consecutive columns of row m) is rounded
// to bf16 and, with a residual, added to the residual row in fp32 and rounded again -- the roundings
// of `residual + linear(x)` on bf16 tensors.  Gated form (a gated MLP's up projection): the weight
// has 2N rows; output column n is h = bf16(bf16(silu(g)) * u) of g = bf16(row n . x) and
// u = bf16(row N + n . x), the roundings of `silu(gate) * up` after `linear(x).chunk(2, -1)` on bf16
// tensors.  Normed form (the block's RMSNorm ahead of the projection): each token row enters as
// bf16(x * r * w_norm) with r = 1 / sqrt(mean(x^2) + eps) -- the rounding of a bf16 nn.RMSNorm -- the
// row's sum of squares formed from the fragments every wave already holds (lane shuffles across the
// four lane groups of a row, then one LDS exchange across the waves).
// ===========================================================================
constexpr int kDlWaves = 16, kDlMaxSteps = 8;  // K <= 16 * 8 * 32 = 4096
constexpr int kDlMaxSplits = 8;

// Split contraction (plain form only): workgroup (b, s) of a (blocks, S) grid takes the 32-wide
// steps [s sps, (s + 1) sps) of column block b and leaves its 16 x 16 partial tile in part (fp32,
// [S][blocks][256]) with device-scope stores; the last of the block's S workgroups to count itself in
// cnt[b] (an atomic increment: it sees S - 1) adds the S tiles in split order -- the same order
// whichever arrives last, so the result does not depend on timing -- finishes the block, and
// returns cnt[b] to zero.  No workgroup waits for another.
struct DlSplit {
  int S, sps;
  float* part;
  unsigned* cnt;
};
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Convolution epilogue (a CCQ-GDN layer's input projections in a decode step, ahead of its decode
// kernels): the q, k and v column blocks leave as bf16(SiLU(short convolution)) of the projection,
// rounded to bf16 first, over the sequence's last kConvW inputs (earlier tokens of the call from the
// lanes holding their rows, older ones from the caches, which the call's last token advances), and
// the a and b columns also give g = -exp(A_log) softplus(a + dt_bias) and beta = sigmoid(b) (x 2
// with negative eigenvalues) -- the per-channel part of the decode prologue, with its roundings;
// the per-head L2 normalisation and lambda, which need whole heads, are left to the decode kernels.
constexpr int kConvW = 4;
struct DlConv {
  int oq, ok, ov, oa, ob;  // first columns of the q (Dq), k (Dq), v (Dv), a (H) and b (H) blocks
  int Dq, Dv, H, T, neg_eig;
  const void *wq, *wk, *wv, *bq, *bk, *bv;  // bf16 [D, kConvW] taps, [D] biases (nullable)
  void *cq, *ck, *cv;                       // bf16 [B, D, kConvW - 1] caches
  const void *alog, *dtb;                   // bf16 [H]
  float *g, *beta;                          // fp32 [M, H]
};

// Gated-norm form (a layer's gated output norm folded into its output projection, the contraction
// split so that each workgroup's steps are exactly one head of dv columns): each operand element
// enters as bf16(x r w[k mod dv] silu(g)) with r = 1 / sqrt(mean of x^2 over the head + eps) from the
// workgroup's own fragments, and the gate g read in place (row stride ldg) -- the arithmetic of the
// gated RMSNorm kernel.
struct DlGate {
  const void* g;   // bf16 gate rows
  long ldg;
  const float* w;  // fp32 [dv] (nullable: ones)
  int dv;
};

// SPW: 32-wide steps per wave (every wave takes SPW; steps past its range read the range's last
// step's address and contribute a zero x fragment, so the code has no branch around a load or an MFMA).
// NT: 16-column tiles per workgroup (plain and normed forms, unsplit): a wide output (an LM head's)
// then has all of its weight loads in flight in one round of workgroups instead of several; wave t
// finishes tile t.
template <int SPW, bool GLU, bool NORM, bool CONV = false, bool GN = false, int NT = 1>
__global__ __launch_bounds__(kDlWaves * 64) void decode_linear_kernel(const void* x_, long ldx, const void* w_,
                                                                       const void* r_, long ldr, void* y_, long ldy,
                                                                       int M, int K, int N, const void* nw_,
                                                                       float eps, const DlSplit sp, const DlConv cv,
                                                                       const DlGate gt) {
  static_assert(NT == 1 || (!GLU && !CONV && !GN), "column tiles: plain and normed forms");
  __shared__ f32x4 sAcc[GLU ? 2 : NT][kDlWaves][64];
  __shared__ float sSS[NORM || GN ? kDlWaves : 1][16];
  const bf16* x = (const bf16*)x_;
  const bf16* w = (const bf16*)w_;
  const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63;
  const int n0 = blockIdx.x * 16 * NT;
  const int s0 = blockIdx.y * sp.sps, steps = min(K / 32, s0 + sp.sps);  // this workgroup's steps [s0, steps)
  const int nw = min(n0 + (l & 15), N - 1);            // weight row of this lane (rows past N repeat the last)
  const int mx = min(l & 15, M - 1);                    // token row of this lane (rows past M repeat the last)
  const bf16* wr = w + (long)nw * K + 8 * (l >> 4);
  auto wrow = [&](int t) { return t == 0 ? wr : w + (long)min(n0 + 16 * t + (l & 15), N - 1) * K + 8 * (l >> 4); };
  const bf16* wu = w + (long)(GLU ? N + nw : nw) * K + 8 * (l >> 4);  // the up half's row (gated form)
  const bf16* xr = x + (long)mx * ldx + 8 * (l >> 4);
  // every load of the wave is issued before the first use
  bf16x8 wa[NT][SPW], wb[GLU ? SPW : 1], xb[SPW], gw[NORM || GN ? SPW : 1];
  f32x4 gn0[GN ? SPW : 1], gn1[GN ? SPW : 1];  // gated-norm form: the norm weight of the step's columns
  const bf16* nr = (const bf16*)(NORM ? nw_ : w_) + 8 * (l >> 4);
  const bf16* gr = GN ? (const bf16*)gt.g + (long)mx * gt.ldg + 8 * (l >> 4) : x;
#pragma unroll
  for (int j = 0; j < SPW; ++j) {
    const int st = min(s0 + wv + kDlWaves * j, steps - 1);
#pragma unroll
    for (int t = 0; t < NT; ++t) wa[t][j] = *gmem((const bf16x8*)(wrow(t) + 32 * st));
    if constexpr (GLU) wb[j] = *gmem((const bf16x8*)(wu + 32 * st));
    xb[j] = *gmem((const bf16x8*)(xr + 32 * st));
    if constexpr (NORM) gw[j] = *gmem((const bf16x8*)(nr + 32 * st));
    if constexpr (GN) {
      gw[j] = *gmem((const bf16x8*)(gr + 32 * st));  // the gate
      const int kh = 32 * (st - s0) + 8 * (l >> 4);  // column within the head
      if (gt.w) {
        gn0[j] = *gmem((const f32x4*)(gt.w + kh));
        gn1[j] = *gmem((const f32x4*)(gt.w + kh + 4));
      } else {
        gn0[j] = gn1[j] = f32x4{1.f, 1.f, 1.f, 1.f};
      }
    }
  }
  float rs = 1.f;
  if constexpr (NORM || GN) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      const bool live = s0 + wv + kDlWaves * j < steps;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = (float)xb[j][i];
        ss += live ? v * v : 0.f;
      }
    }
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    if (l < 16) sSS[wv][l] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int q = 0; q < kDlWaves; ++q) tot += sSS[q][l & 15];
    rs = rsqrtf(tot / (float)(GN ? gt.dv : K) + eps);
  }
  f32x4 acc[NT], acu = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = acu;
#pragma unroll
  for (int j = 0; j < SPW; ++j) {
    const bool live = s0 + wv + kDlWaves * j < steps;
    bf16x8 xf;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      bf16 v = xb[j][i];
      if constexpr (NORM) v = (bf16)((float)v * rs * (float)gw[j][i]);
      if constexpr (GN) {
        const float g = (float)gw[j][i], wn = i < 4 ? gn0[j][i] : gn1[j][i - 4];
        v = (bf16)((float)v * rs * wn * (g / (1.f + __expf(-g))));
      }
      xf[i] = live ? v : (bf16)0.f;
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = mfma16(wa[t][j], xf, acc[t]);
    if constexpr (GLU) acu = mfma16(wb[j], xf, acu);
  }
  // convolution epilogue: thread (row tid / 16, column tid % 16) of the first four waves takes one
  // result; its column's taps, bias, its row's cache window and the gate constants are loaded after
  // the products, while the other waves finish theirs
  const int er = tid >> 4, ec = tid & 15;
  int ekind = 0, ech = 0;  // column kind (0 none, 1 q, 2 k, 3 v, 4 a, 5 b) and channel / head
  float cw[CONV ? kConvW : 1], cb = 0.f, cc[CONV ? kConvW - 1 : 1], ca = 0.f, cd = 0.f;
  if constexpr (CONV) {
    const int n = n0 + ec;
    if (n >= cv.oq && n < cv.oq + cv.Dq) { ekind = 1; ech = n - cv.oq; }
    else if (n >= cv.ok && n < cv.ok + cv.Dq) { ekind = 2; ech = n - cv.ok; }
    else if (n >= cv.ov && n < cv.ov + cv.Dv) { ekind = 3; ech = n - cv.ov; }
    else if (n >= cv.oa && n < cv.oa + cv.H) { ekind = 4; ech = n - cv.oa; }
    else if (n >= cv.ob && n < cv.ob + cv.H) { ekind = 5; ech = n - cv.ob; }
#pragma unroll
    for (int j = 0; j < kConvW; ++j) cw[j] = 0.f;
#pragma unroll
    for (int j = 0; j < kConvW - 1; ++j) cc[j] = 0.f;
    if (tid < 256 && ekind >= 1 && ekind <= 3) {
      const int k = ekind, c = ech, D = k == 3 ? cv.Dv : cv.Dq, b = min(er, M - 1) / cv.T;
      const bf16* tw = (const bf16*)(k == 1 ? cv.wq : k == 2 ? cv.wk : cv.wv) + (long)c * kConvW;
      const bf16* tb = (const bf16*)(k == 1 ? cv.bq : k == 2 ? cv.bk : cv.bv);
      const bf16* tc = (const bf16*)(k == 1 ? cv.cq : k == 2 ? cv.ck : cv.cv) + ((long)b * D + c) * (kConvW - 1);
#pragma unroll
      for (int j = 0; j < kConvW; ++j) cw[j] = (float)tw[j];
      if (tb) cb = (float)tb[c];
#pragma unroll
      for (int j = 0; j < kConvW - 1; ++j) cc[j] = (float)tc[j];
    } else if (tid < 256 && ekind == 4) {
      ca = (float)((const bf16*)cv.alog)[ech];
      cd = (float)((const bf16*)cv.dtb)[ech];
    }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) sAcc[t][wv][l] = acc[t];
  if constexpr (GLU) sAcc[GLU ? 1 : 0][wv][l] = acu;
  __syncthreads();
  if constexpr (CONV) {
    // wave 0: the tile's projection as bf16 values into LDS (row m, column n - n0), for every
    // thread of the first four waves to read its window's earlier rows
    __shared__ float sY[16][17];
    if (wv == 0) {
      f32x4 t4 = sAcc[0][0][l];
#pragma unroll
      for (int q = 1; q < kDlWaves; ++q) {
        const f32x4 v = sAcc[0][q][l];
        t4[0] += v[0]; t4[1] += v[1]; t4[2] += v[2]; t4[3] += v[3];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) sY[l & 15][4 * (l >> 4) + i] = (float)(bf16)t4[i];
    }
    __syncthreads();
    if (tid >= 256) return;
    const int m = er, n = n0 + ec;
    if (m >= M || n >= N) return;
    const int b = m / cv.T, t = m - b * cv.T;
    const float yr = sY[m][ec];
    // input d tokens back (d <= t: row m - d of the tile; else cache slot kConvW - 1 + t - d)
    auto input = [&](int d) {
      float v = d == 0 ? yr : 0.f;
#pragma unroll
      for (int q = 0; q < kConvW - 1; ++q)
        if (d > t && q == kConvW - 1 + t - d) v = cc[q];
#pragma unroll
      for (int e = 1; e < kConvW; ++e)
        if (d == e && e <= t) v = sY[m - e][ec];
      return v;
    };
    float out = yr;
    if (ekind >= 1 && ekind <= 3) {
      float acc2 = cb + cw[kConvW - 1] * yr;
#pragma unroll
      for (int j = 0; j < kConvW - 1; ++j) acc2 += cw[j] * input(kConvW - 1 - j);
      out = (float)(bf16)(acc2 / (1.f + __expf(-acc2)));
      if (t == cv.T - 1) {
        // the call's last kConvW - 1 inputs into the cache
        const int D = ekind == 3 ? cv.Dv : cv.Dq;
        bf16* tc = (bf16*)(ekind == 1 ? cv.cq : ekind == 2 ? cv.ck : cv.cv) + ((long)b * D + ech) * (kConvW - 1);
        float nwin[kConvW - 1];
#pragma unroll
        for (int q = 0; q < kConvW - 1; ++q) nwin[q] = input(kConvW - 2 - q);
#pragma unroll
        for (int q = 0; q < kConvW - 1; ++q) tc[q] = (bf16)nwin[q];
      }
    } else if (ekind == 4) {
      const float xa = yr + cd;
      cv.g[(long)m * cv.H + ech] = -expf(ca) * (xa > 20.f ? xa : log1pf(expf(xa)));
    } else if (ekind == 5) {
      float be = (float)(bf16)(1.f / (1.f + expf(-yr)));
      if (cv.neg_eig) be *= 2.f;
      cv.beta[(long)m * cv.H + ech] = be;
    }
    ((bf16*)y_)[(long)m * ldy + n] = (bf16)out;
    return;
  }
  if (wv >= NT) return;
  const int tt = NT > 1 ? wv : 0;  // this wave's tile
  f32x4 sum = sAcc[tt][0][l];
#pragma unroll
  for (int q = 1; q < kDlWaves; ++q) {
    const f32x4 v = sAcc[tt][q][l];
    sum[0] += v[0]; sum[1] += v[1]; sum[2] += v[2]; sum[3] += v[3];
  }
  if (sp.S > 1) {
    // this split's tile out, counted in; the last to arrive adds the S tiles in split order
    float* const part = sp.part + (long)blockIdx.x * 256 + 4 * l;
    const long pstride = (long)gridDim.x * 256;
#pragma unroll
    for (int i = 0; i < 4; ++i) st_dev(part + blockIdx.y * pstride + i, sum[i]);
    __builtin_amdgcn_s_waitcnt(0);  // the stores acknowledged before the count
    unsigned old = 0;
    if (l == 0) old = __hip_atomic_fetch_add(sp.cnt + blockIdx.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __builtin_amdgcn_readfirstlane(old);
    if (old != (unsigned)(sp.S - 1)) return;
    f32x4 tot = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int q = 0; q < sp.S; ++q) {
#pragma unroll
      for (int i = 0; i < 4; ++i) tot[i] += q == (int)blockIdx.y ? sum[i] : ld_dev(part + q * pstride + i);
    }
    sum = tot;
    if (l == 0) __hip_atomic_store(sp.cnt + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if constexpr (GLU) {
    f32x4 su = sAcc[GLU ? 1 : 0][0][l];
#pragma unroll
    for (int q = 1; q < kDlWaves; ++q) {
      const f32x4 v = sAcc[GLU ? 1 : 0][q][l];
      su[0] += v[0]; su[1] += v[1]; su[2] += v[2]; su[3] += v[3];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float g = (float)(bf16)sum[i];
      sum[i] = (float)(bf16)(g / (1.f + expf(-g))) * (float)(bf16)su[i];  // rounded once more at the store
    }
  }
  // sum[i] = y[m = l & 15][n = n0 + 16 tt + 4 (l >> 4) + i]
  const int m = l & 15, nb = n0 + 16 * tt + 4 * (l >> 4);
  if (m >= M) return;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int n = nb + i;
    if (n < N) {
      float v = GLU ? sum[i] : (float)(bf16)sum[i];
      if (r_) v += (float)((const bf16*)r_)[(long)m * ldr + n];
      ((bf16*)y_)[(long)m * ldy + n] = (bf16)v;
    }
  }
}

// Column tiles per workgroup of a wide plain or normed projection: four when that still leaves 200
// workgroups or more (an LM head's 32,000 columns: 500 workgroups, 21.6 us for 65.5 MB at 16 tokens
// against 26.1 us with one tile; eight tiles measured the same as four).
constexpr int kDlWideTiles = 4;
inline bool dl_wide(bool glu, int blocks, const DlSplit& sp, const DlConv* conv, const DlGate* gate) {
  return !glu && !conv && !gate && sp.S == 1 && blocks >= 200 * kDlWideTiles;
}

template <int SPW>
static void launch_dl(bool glu, dim3 grid, dim3 block, hipStream_t st, const void* x, long ldx, const void* w,
                      const void* r, long ldr, void* y, long ldy, int M, int K, int N, const void* nw, float eps,
                      const DlSplit& sp, const DlConv* conv, const DlGate* gate) {
  const DlConv cv = conv ? *conv : DlConv{};
  const DlGate gt = gate ? *gate : DlGate{};
  // (contractions up to 1024: the tiles of longer ones would spill)
  if (SPW <= 2 && dl_wide(glu, (int)grid.x, sp, conv, gate)) {
    constexpr int S2 = SPW <= 2 ? SPW : 1;  // (no instances for longer contractions)
    const dim3 g4((grid.x + kDlWideTiles - 1) / kDlWideTiles, 1);
    if (nw)
      hipLaunchKernelGGL((decode_linear_kernel<S2, false, true, false, false, kDlWideTiles>), g4, block, 0, st, x, ldx,
                         w, r, ldr, y, ldy, M, K, N, nw, eps, sp, cv, gt);
    else
      hipLaunchKernelGGL((decode_linear_kernel<S2, false, false, false, false, kDlWideTiles>), g4, block, 0, st, x,
                         ldx, w, r, ldr, y, ldy, M, K, N, nw, eps, sp, cv, gt);
    return;
  }
#define CCQ_DL(G, NM)                                                                                        \
  hipLaunchKernelGGL((decode_linear_kernel<SPW, G, NM>), grid, block, 0, st, x, ldx, w, r, ldr, y, ldy, M, K, N, \
                     nw, eps, sp, cv, gt)
  if (gate) {
    hipLaunchKernelGGL((decode_linear_kernel<SPW, false, false, false, true>), grid, block, 0, st, x, ldx, w, r, ldr,
                       y, ldy, M, K, N, nw, eps, sp, cv, gt);
  } else if (conv) {
    if (nw)
      hipLaunchKernelGGL((decode_linear_kernel<SPW, false, true, true>), grid, block, 0, st, x, ldx, w, r, ldr, y,
                         ldy, M, K, N, nw, eps, sp, cv, gt);
    else
      hipLaunchKernelGGL((decode_linear_kernel<SPW, false, false, true>), grid, block, 0, st, x, ldx, w, r, ldr, y,
                         ldy, M, K, N, nw, eps, sp, cv, gt);
  } else if (glu) {
    if (nw) CCQ_DL(true, true); else CCQ_DL(true, false);
  } else {
    if (nw) CCQ_DL(false, true); else CCQ_DL(false, false);
  }
#undef CCQ_DL
}

// Workspace of the split form: the block counters (zero between calls), then the partial tiles.
size_t decode_linear_split_bytes(int N, int splits) {
  const size_t blocks = (size_t)(N + 15) / 16;
  return ((blocks * 4 + 255) / 256) * 256 + (size_t)splits * blocks * 256 * 4;
}

hipError_t launch_decode_linear(bool glu, const void* x, long ldx, const void* w, const void* r, long ldr, void* y,
                                long ldy, int M, int K, int N, const void* nw, float eps, int splits, void* ws,
                                const DlConv* conv, hipStream_t st, const DlGate* gate) {
  if (M <= 0 || N <= 0) return hipSuccess;
  const int blocks = (N + 15) / 16, steps = K / 32;
  DlSplit sp{1, steps, nullptr, nullptr};
  if (splits > 1) {
    sp.sps = (steps + splits - 1) / splits;
    sp.S = (steps + sp.sps - 1) / sp.sps;  // (no empty split)
    sp.cnt = (unsigned*)ws;
    sp.part = (float*)((char*)ws + ((size_t)blocks * 4 + 255) / 256 * 256);
  }
  const dim3 grid((unsigned)blocks, (unsigned)sp.S), block(kDlWaves * 64);
  const int spw = (sp.sps + kDlWaves - 1) / kDlWaves;
  switch (spw) {
    case 1: launch_dl<1>(glu, grid, block, st, x, ldx, w, r, ldr, y, ldy, M, K, N, nw, eps, sp, conv, gate); break;
    case 2: launch_dl<2>(glu, grid, block, st, x, ldx, w, r, ldr, y, ldy, M, K, N, nw, eps, sp, conv, gate); break;
    case 3: launch_dl<3>(glu, grid, block, st, x, ldx, w, r, ldr, y, ldy, M, K, N, nw, eps, sp, conv, gate); break;
    case 4: launch_dl<4>(glu, grid, block, st, x, ldx, w, r, ldr, y, ldy, M, K, N, nw, eps, sp, conv, gate); break;
    case 5: launch_dl<5>(glu, grid, block, st, x, ldx, w, r, ldr, y, ldy, M, K, N, nw, eps, sp, conv, gate); break;
    case 6: launch_dl<6>(glu, grid, block, st, x, ldx, w, r, ldr, y, ldy, M, K, N, nw, eps, sp, conv, gate); break;
    case 7: launch_dl<7>(glu, grid, block, st, x, ldx, w, r, ldr, y, ldy, M, K, N, nw, eps, sp, conv, gate); break;
    case 8: launch_dl<8>(glu, grid, block, st, x, ldx, w, r, ldr, y, ldy, M, K, N, nw, eps, sp, conv, gate); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_decode_in_proj(const void* x, long ldx, const void* w, void* y, long ldy, int M, int K, int N,
                                 const void* nw, float eps, int oq, int ok, int ov, int oa, int ob, int Dq, int Dv,
                                 int H, int T, int neg_eig, const void* wq, const void* wk, const void* wv,
                                 const void* bq, const void* bk, const void* bv, void* cq, void* ck, void* cv,
                                 const void* alog, const void* dtb, float* g, float* beta, hipStream_t st) {
  DlConv c{oq, ok, ov, oa, ob, Dq, Dv, H, T, neg_eig, wq, wk, wv, bq, bk, bv, cq, ck, cv, alog, dtb, g, beta};
  return launch_decode_linear(false, x, ldx, w, nullptr, 0, y, ldy, M, K, N, nw, eps, 1, nullptr, &c, st, nullptr);
}

// The output projection with the gated output norm folded in: the contraction split per head (K / dv
// workgroups per column block, one head each).
hipError_t launch_decode_linear_gnorm(const void* x, long ldx, const void* g, long ldg, const float* gw, int dv,
                                      float geps, const void* w, const void* r, long ldr, void* y, long ldy, int M,
                                      int K, int N, void* ws, hipStream_t st) {
  const DlGate gt{g, ldg, gw, dv};
  return launch_decode_linear(false, x, ldx, w, r, ldr, y, ldy, M, K, N, nullptr, geps, K / dv, ws, nullptr, st, &gt);
}

// ===========================================================================
// Greedy step of a generate loop: ids[m] = argmax_n logits[m][n] (the first index of the maximum; a
// NaN counts as larger than any number, the first NaN winning, as torch.argmax), then the embedding
// row of that token into x[m] (zeros for an id past the table's rows) -- the next decode step's input,
// gathered here so that the step needs no launch of its own for it.  One workgroup per row: each
// thread scans 8-element pieces (16-byte loads, for aligned rows) strided across the row, the wave's
// best by lane exchanges, the workgroup's through LDS.
// ===========================================================================
constexpr int kGreedyThreads = 1024;

__device__ __forceinline__ bool greedy_better(float v, int i, float u, int j) {
  const bool nv = v != v, nu = u != u;
  if (nv != nu) return nv;
  if (!nv && v != u) return v > u;
  return i < j;
}

// vec: rows 16-byte aligned (pieces of 8 elements; else every element by itself)
__global__ __launch_bounds__(kGreedyThreads) void greedy_embed_kernel(const bf16* logits, long ldl, int N, bool vec,
                                                                      const bf16* table, long rows, int D,
                                                                      int64_t* ids, long ldi, bf16* x, long ldx) {
  __shared__ float sv[kGreedyThreads / 64];
  __shared__ int si[kGreedyThreads / 64];
  __shared__ int sbest;
  const int m = blockIdx.x, tid = threadIdx.x;
  const bf16* row = logits + (long)m * ldl;
  float bv = -__builtin_inff();
  int bi = N;  // (no element yet: loses to any element)
  // PB pieces per thread in flight at once (unconditional loads from clamped addresses; a loop of
  // one load per pass would wait for each)
  constexpr int PB = 4;
  const int n8 = vec ? N / 8 : 0;
  for (int p0 = 0; p0 < n8; p0 += PB * kGreedyThreads) {
    bf16x8 v[PB];
#pragma unroll
    for (int b = 0; b < PB; ++b) v[b] = *(const bf16x8*)(row + 8 * min(p0 + b * kGreedyThreads + tid, n8 - 1));
#pragma unroll
    for (int b = 0; b < PB; ++b) {
      const int p = p0 + b * kGreedyThreads + tid;
      if (p < n8) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (greedy_better((float)v[b][e], 8 * p + e, bv, bi)) {
            bv = (float)v[b][e];
            bi = 8 * p + e;
          }
      }
    }
  }
  for (int n = 8 * n8 + tid; n < N; n += kGreedyThreads)
    if (greedy_better((float)row[n], n, bv, bi)) {
      bv = (float)row[n];
      bi = n;
    }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float u = __shfl_xor(bv, o);
    const int j = __shfl_xor(bi, o);
    if (greedy_better(u, j, bv, bi)) {
      bv = u;
      bi = j;
    }
  }
  if ((tid & 63) == 0) {
    sv[tid >> 6] = bv;
    si[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kGreedyThreads / 64; ++w)
      if (greedy_better(sv[w], si[w], bv, bi)) {
        bv = sv[w];
        bi = si[w];
      }
    ids[(long)m * ldi] = bi;
    sbest = bi;
  }
  __syncthreads();
  const long id = sbest;
  const bf16* src = table + id * D;
  bf16* dst = x + (long)m * ldx;
  const bool ok = id < rows;
  for (int c = tid; c < D; c += kGreedyThreads) dst[c] = ok ? src[c] : (bf16)0.f;
}

hipError_t launch_greedy_embed(const void* logits, long ldl, int M, int N, const void* table, long rows, int D,
                               int64_t* ids, long ldi, void* x, long ldx, hipStream_t st) {
  if (M <= 0) return hipSuccess;
  const bool vec = ((uintptr_t)logits & 15) == 0 && ldl % 8 == 0;
  hipLaunchKernelGGL(greedy_embed_kernel, dim3(M), dim3(kGreedyThreads), 0, st, (const bf16*)logits, ldl, N, vec,
                     (const bf16*)table, rows, D, ids, ldi, (bf16*)x, ldx);
  return hipGetLastError();
}

hipError_t launch_decode(const DecodeArgs& a, hipStream_t st) {
  if (a.N <= 0 || a.H <= 0) return hipSuccess;
  switch (a.K) {
    case 32: return launch_decode_k<32>(a, st);
    case 64: return launch_decode_k<64>(a, st);
    case 128: return launch_decode_k<128>(a, st);
    case 256: return launch_decode_k<256>(a, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ccq
