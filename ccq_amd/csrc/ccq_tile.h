// Shared device-side building blocks for the CCQ HIP kernels (gfx950 / CDNA4).
//
// Every matrix product in this library is a 32x32 output tile computed by one
// 64-lane wavefront with v_mfma_f32_32x32x16_bf16 (fp32 accumulate).  Operand
// fragments come from LDS.  Lane layout of that instruction (checked on the
// device by the GPU parity tests in tests/):
//   A (32 x 16, rows x contraction):  lane l holds row l%32, k = 8*(l/32) .. +7
//   B (16 x 32, contraction x cols):  lane l holds col l%32, k = 8*(l/32) .. +7
//   C (32 x 32):                      lane l holds col l%32, rows
//                                     8*(i/4) + 4*(l/32) + i%4 for i = 0..15
//
// fp32 operands that must keep more than bf16's 8 significant bits are fed as
// a hi/lo pair (x = hi + lo, both bf16) and cost two or three MFMAs.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ccq {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x8 __attribute__((ext_vector_type(8)));  // int16 bit patterns of a 16-byte piece
typedef short s16x4 __attribute__((ext_vector_type(4)));  // int16 values of an 8-byte piece
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;  // 4 wavefronts per workgroup
constexpr int kWalk8 = 512;    // 8 wavefronts: the walks with separate compute and memory waves

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// Row / column inside a 32x32 accumulator tile of element i held by this lane.
__device__ __forceinline__ int acc_row(int i) { return ((i >> 2) << 3) + ((lane_id() >> 5) << 2) + (i & 3); }
__device__ __forceinline__ int acc_col() { return lane_id() & 31; }

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

__device__ __forceinline__ f32x16 mfma(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// 16x16 output tiles with v_mfma_f32_16x16x32_bf16:
//   A (16 x 32):  lane l holds row l%16, k = 8*(l/16) .. +7
//   B (32 x 16):  lane l holds col l%16, k = 8*(l/16) .. +7
//   C (16 x 16):  lane l holds col l%16, rows 4*(l/16) + i for i = 0..3
__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Global-memory view of a pointer.  Pointers cast from void* are not always inferred as global, and
// a flat access also holds the LDS wait counter; spelling the address space keeps global_* code.
template <class T>
__device__ __forceinline__ __attribute__((address_space(1))) T* gmem(T* p) {
  return (__attribute__((address_space(1))) T*)p;
}
template <class T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gmem(const T* p) {
  return (const __attribute__((address_space(1))) T*)p;
}

__device__ __forceinline__ bf16 to_bf16(float x) { return (bf16)x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }

__device__ __forceinline__ void split2(float x, bf16& hi, bf16& lo) {
  hi = (bf16)x;
  lo = (bf16)(x - (float)hi);
}

// ---------------------------------------------------------------------------
// fragment loaders.  `p` points at element (row 0, k 0) of the 32-row slab.
// ---------------------------------------------------------------------------

// Element (r, k) at p[r * ld + k]  (contraction index contiguous: one 16-byte read).
__device__ __forceinline__ bf16x8 frag_rm(const bf16* p, int ld) {
  const int l = lane_id();
  return *(const bf16x8*)(p + (l & 31) * ld + ((l >> 5) << 3));
}

// 16x32 operand of mfma16, element (r, k) at p[r * ld + k] (one 16-byte read).
__device__ __forceinline__ bf16x8 frag16_rm(const bf16* p, int ld) {
  const int l = lane_id();
  return *(const bf16x8*)(p + (l & 15) * ld + ((l >> 4) << 3));
}

// 16x32 operand of mfma16 whose contraction index runs down the rows of a row-major tile: element
// (r, k) at p[k * ld + r].  Two transposing LDS reads (ds_read_b64_tr_b16): in each 16-lane group,
// lane j names the 8-byte piece at row (j >> 2), columns 4 (j & 3) .. +3 of a 4 x 16 block, and lane
// i receives column i of the block -- four consecutive contraction elements of operand row i.
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ bf16x8 frag16_tr(const bf16* p, int ld) {
  const int l = lane_id(), j = l & 15;
  const bf16* q = p + (8 * (l >> 4) + (j >> 2)) * ld + 4 * (j & 3);
  typedef __attribute__((address_space(3))) bf16x4_t lds_b4;
  const bf16x4_t a = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_b4*)q);
  const bf16x4_t b = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_b4*)(q + 4 * ld));
  return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Buffer resource over `bytes` bytes from p (gfx9 raw buffer, stride 0): a buffer store whose byte
// offset is at or beyond `bytes` is dropped by the hardware, so rows past a chunk can be stored
// without a branch (a branch lets the compiler sink the loads that feed the stored values into it).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, 0x00020000);
}

// 32x16 operand of mfma (32x32x16) whose contraction index runs down the rows of a row-major tile:
// element (r, k) at p[k * ld + r].  Two transposing LDS reads; 16-lane group g covers operand rows
// 16 (g & 1) .. +15 and contraction elements 8 (g >> 1) .. +7 (lane j of the group names the 8-byte
// piece at row j >> 2, columns 4 (j & 3) .. +3 of its 4 x 16 block).
__device__ __forceinline__ bf16x8 frag32_tr(const bf16* p, int ld) {
  const int l = lane_id(), j = l & 15;
  const bf16* q = p + (8 * (l >> 5) + (j >> 2)) * ld + 16 * ((l >> 4) & 1) + 4 * (j & 3);
  typedef __attribute__((address_space(3))) bf16x4_t lds_b4;
  const bf16x4_t a = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_b4*)q);
  const bf16x4_t b = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_b4*)(q + 4 * ld));
  return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Element (r, k) at p[k * ld + r]  (operand stored transposed: eight 2-byte reads).
__device__ __forceinline__ bf16x8 frag_cm(const bf16* p, int ld) {
  const int l = lane_id();
  const bf16* q = p + ((l >> 5) << 3) * ld + (l & 31);
  bf16x8 v;
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = q[i * ld];
  return v;
}

// fp32 operand, element (r, k) at p[r * ld + k], split into hi/lo on the fly.
__device__ __forceinline__ void frag_rm_f32(const float* p, int ld, bf16x8& hi, bf16x8& lo) {
  const int l = lane_id();
  const float* q = p + (l & 31) * ld + ((l >> 5) << 3);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    bf16 h, o;
    split2(q[i], h, o);
    hi[i] = h;
    lo[i] = o;
  }
}

// fp32 operand, element (r, k) at p[k * ld + r], split into hi/lo on the fly.
__device__ __forceinline__ void frag_cm_f32(const float* p, int ld, bf16x8& hi, bf16x8& lo) {
  const int l = lane_id();
  const float* q = p + ((l >> 5) << 3) * ld + (l & 31);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    bf16 h, o;
    split2(q[i * ld], h, o);
    hi[i] = h;
    lo[i] = o;
  }
}

// fp32 operand element (r, k) at p[r * ld + k] scaled by ks[k] (scale indexed by the contraction
// index), split into hi/lo on the fly.
__device__ __forceinline__ void frag_rm_f32_ks(const float* p, int ld, const float* ks, bf16x8& hi, bf16x8& lo) {
  const int l = lane_id();
  const int kb = (l >> 5) << 3;
  const float* q = p + (l & 31) * ld + kb;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    bf16 hh, oo;
    split2(q[i] * ks[kb + i], hh, oo);
    hi[i] = hh;
    lo[i] = oo;
  }
}

// 0/1 lower-triangular (inclusive) fragment: element (r, k) = (k <= r), rows offset r0, k offset k0.
__device__ __forceinline__ bf16x8 frag_tril_ones(int r0, int k0) {
  const int l = lane_id();
  const int r = r0 + (l & 31);
  const int kb = k0 + ((l >> 5) << 3);
  bf16x8 v;
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (bf16)((kb + i <= r) ? 1.f : 0.f);
  return v;
}

// 0/1 upper-triangular (inclusive) fragment: element (r, k) = (k >= r).
__device__ __forceinline__ bf16x8 frag_triu_ones(int r0, int k0) {
  const int l = lane_id();
  const int r = r0 + (l & 31);
  const int kb = k0 + ((l >> 5) << 3);
  bf16x8 v;
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (bf16)((kb + i >= r) ? 1.f : 0.f);
  return v;
}

// ---------------------------------------------------------------------------
// whole-contraction helpers: acc += A B over kdim (multiple of 16)
// A: rows from p_a (layout rm or cm), B: columns from p_b (layout rm = [col][k], cm = [k][col])
// ---------------------------------------------------------------------------

// A row-major [r][k], B stored [n][k]
__device__ __forceinline__ void mma_rr(f32x16& acc, const bf16* a, int lda, const bf16* b, int ldb, int kdim) {
  for (int k0 = 0; k0 < kdim; k0 += 16) acc = mfma(frag_rm(a + k0, lda), frag_rm(b + k0, ldb), acc);
}

// A stored [k][r] (transposed), B stored [n][k]
__device__ __forceinline__ void mma_cr(f32x16& acc, const bf16* a, int lda, const bf16* b, int ldb, int kdim) {
  for (int k0 = 0; k0 < kdim; k0 += 16) acc = mfma(frag_cm(a + k0 * lda, lda), frag_rm(b + k0, ldb), acc);
}

// A stored [r][k], B stored [k][n] (transposed)
__device__ __forceinline__ void mma_rc(f32x16& acc, const bf16* a, int lda, const bf16* b, int ldb, int kdim) {
  for (int k0 = 0; k0 < kdim; k0 += 16) acc = mfma(frag_rm(a + k0, lda), frag_cm(b + k0 * ldb, ldb), acc);
}

// ---------------------------------------------------------------------------
// global -> LDS tile staging (rows of a token-major tensor)
// ---------------------------------------------------------------------------

// Copy `rows` rows of D bf16 each (row r at g[r * gstride]) into LDS (row-major, leading dim ld)
// and optionally a transposed copy (dst_t[c * ldt + r]).  Rows >= nvalid are zero-filled.
template <int D>
__device__ __forceinline__ void stage_bf16(bf16* dst, int ld, bf16* dst_t, int ldt, const bf16* g, long gstride,
                                           int rows, int nvalid) {
  constexpr int VPR = D / 8;
  for (int idx = threadIdx.x; idx < rows * VPR; idx += kThreads) {
    const int r = idx / VPR, c = (idx % VPR) * 8;
    bf16x8 v;
    if (r < nvalid) {
      v = *(const bf16x8*)(g + (long)r * gstride + c);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = (bf16)0.f;
    }
    if (dst) *(bf16x8*)(dst + r * ld + c) = v;
    if (dst_t) {
#pragma unroll
      for (int i = 0; i < 8; ++i) dst_t[(c + i) * ldt + r] = v[i];
    }
  }
}

// Same for fp32 rows into fp32 LDS (row-major and/or transposed).
template <int D>
__device__ __forceinline__ void stage_f32(float* dst, int ld, float* dst_t, int ldt, const float* g, long gstride,
                                          int rows, int nvalid) {
  constexpr int VPR = D / 4;
  for (int idx = threadIdx.x; idx < rows * VPR; idx += kThreads) {
    const int r = idx / VPR, c = (idx % VPR) * 4;
    f32x4 v;
    if (r < nvalid) {
      v = *(const f32x4*)(g + (long)r * gstride + c);
    } else {
      v[0] = v[1] = v[2] = v[3] = 0.f;
    }
    if (dst) {
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[r * ld + c + i] = v[i];
    }
    if (dst_t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) dst_t[(c + i) * ldt + r] = v[i];
    }
  }
}


// Stage ROWS x D bf16 rows into a transposed LDS tile dst_t[c * ldt + r] (ldt % 4 == 0).  Each
// thread reads a 4-row x 8-column patch and writes eight 4-element (8-byte) column pieces; lanes
// that share a column sit on consecutive rows, so the 8-byte writes hit consecutive banks.
template <int D, int ROWS>
__device__ __forceinline__ void stage_bf16_t4(bf16* dst_t, int ldt, const bf16* g, long gstride, int nvalid) {
  constexpr int RG = ROWS / 4, CG = D / 8;
  for (int idx = threadIdx.x; idx < RG * CG; idx += kThreads) {
    const int rg = idx % RG, cg = idx / RG;
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
      typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
      bf16x4 col;
      col[0] = v[0][i];
      col[1] = v[1][i];
      col[2] = v[2][i];
      col[3] = v[3][i];
      *(bf16x4*)(dst_t + (c0 + i) * ldt + r0) = col;
    }
  }
}

// fp32 operand stored row-major, read transposed: element (r, k) at p[k * ld + r] scaled by ks[k]
// (scale indexed by the contraction index), split into hi/lo.
__device__ __forceinline__ void frag_cm_f32_ks(const float* p, int ld, const float* ks, bf16x8& hi, bf16x8& lo) {
  const int l = lane_id();
  const int kb = (l >> 5) << 3;
  const float* q = p + kb * ld + (l & 31);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    bf16 hh, oo;
    split2(q[i * ld] * ks[kb + i], hh, oo);
    hi[i] = hh;
    lo[i] = oo;
  }
}

// Sequence bounds for dense ([B, T]) or varlen (B == 1 + cu_seqlens) inputs.
__device__ __forceinline__ void seq_bounds(const int64_t* cu, int n, int T, long& bos, int& len) {
  if (cu) {
    bos = (long)cu[n];
    len = (int)(cu[n + 1] - cu[n]);
  } else {
    bos = (long)n * T;
    len = T;
  }
}

// Workgroups are handed to the 8 XCDs round-robin by linear id.  Give the `nsplit`
// workgroups that share one (sequence, head) the same XCD so they share its L2.
__device__ __forceinline__ void xcd_map(int bid, int nsplit, int nunits, int& unit, int& split) {
  if ((nunits & 7) == 0) {
    const int xcd = bid & 7, slot = bid >> 3;
    split = slot % nsplit;
    unit = (slot / nsplit) * 8 + xcd;
  } else {
    split = bid % nsplit;
    unit = bid / nsplit;
  }
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.f / (1.f + __expf(-x)); }


// ---------------------------------------------------------------------------
// register prefetch of a ROWS x D tile (one step ahead of its use)
// ---------------------------------------------------------------------------

template <int D, int ROWS>
struct PrefetchBf16 {
  static constexpr int VPR = D / 8;
  static constexpr int N = (ROWS * VPR + kThreads - 1) / kThreads;
  bf16x8 v[N];
  __device__ __forceinline__ void load(const bf16* g, long gstride, int nvalid) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = threadIdx.x + j * kThreads;
      const int r = idx / VPR, c = (idx % VPR) * 8;
      if (idx < ROWS * VPR && r < nvalid) {
        v[j] = *(const bf16x8*)(g + (long)r * gstride + c);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[j][i] = (bf16)0.f;
      }
    }
  }
  __device__ __forceinline__ void store(bf16* dst, int ld, bf16* dst_t, int ldt) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = threadIdx.x + j * kThreads;
      if (idx >= ROWS * VPR) continue;
      const int r = idx / VPR, c = (idx % VPR) * 8;
      if (dst) *(bf16x8*)(dst + r * ld + c) = v[j];
      if (dst_t) {
#pragma unroll
        for (int i = 0; i < 8; ++i) dst_t[(c + i) * ldt + r] = v[j][i];
      }
    }
  }
  // The pieces hold int16 rows of a block-floating-point tile (each row an integer vector times a
  // power-of-two scale): the scale of each piece's row from `scales` (one per row, nvalid rows)
  __device__ __forceinline__ void load_scales(const float* scales, int nvalid, float (&sc)[N]) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = threadIdx.x + j * kThreads, r = idx / VPR;
      sc[j] = (idx < ROWS * VPR && r < nvalid) ? scales[r] : 0.f;
    }
  }
  // row-major copy of scale x integer as a hi/lo pair (exact: the value has at most 16 significant bits)
  __device__ __forceinline__ void store_s16_split(bf16* hi, bf16* lo, int ld, const float (&sc)[N]) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = threadIdx.x + j * kThreads;
      if (idx >= ROWS * VPR) continue;
      const int r = idx / VPR, c = (idx % VPR) * 8;
      // reinterpret the whole piece: a bit cast of one vector element reads element 0 here
      const s16x8 x = __builtin_bit_cast(s16x8, v[j]);
      bf16x8 h8, l8;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        bf16 a, b;
        split2(sc[j] * (float)x[i], a, b);
        h8[i] = a;
        l8[i] = b;
      }
      *(bf16x8*)(hi + r * ld + c) = h8;
      *(bf16x8*)(lo + r * ld + c) = l8;
    }
  }
};

template <int D, int ROWS>
struct PrefetchF32 {
  static constexpr int VPR = D / 4;
  static constexpr int N = (ROWS * VPR + kThreads - 1) / kThreads;
  f32x4 v[N];
  __device__ __forceinline__ void load(const float* g, long gstride, int nvalid) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = threadIdx.x + j * kThreads;
      const int r = idx / VPR, c = (idx % VPR) * 4;
      if (idx < ROWS * VPR && r < nvalid) {
        v[j] = *(const f32x4*)(g + (long)r * gstride + c);
      } else {
        v[j][0] = v[j][1] = v[j][2] = v[j][3] = 0.f;
      }
    }
  }
  // bf16 source promoted to fp32 (8 elements per vector -> two f32x4 per thread slot)
  __device__ __forceinline__ void store(float* dst, int ld, float* dst_t, int ldt) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = threadIdx.x + j * kThreads;
      if (idx >= ROWS * VPR) continue;
      const int r = idx / VPR, c = (idx % VPR) * 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (dst) dst[r * ld + c + i] = v[j][i];
        if (dst_t) dst_t[(c + i) * ldt + r] = v[j][i];
      }
    }
  }
};

// A gradient input that may arrive as fp32 or bf16 rows, staged into fp32 LDS.
template <int D, int ROWS>
struct PrefetchGrad {
  PrefetchF32<D, ROWS> f;
  PrefetchBf16<D, ROWS> b;
  __device__ __forceinline__ void load(const float* g32, const bf16* g16, long gstride, int nvalid) {
    if (g32) f.load(g32, gstride, nvalid);
    else b.load(g16, gstride, nvalid);
  }
  // row-major (dst[r * ld + c]) and/or transposed (dst_t[c * ldt + r]) fp32 copies
  __device__ __forceinline__ void store(bool is32, float* dst, int ld, float* dst_t = nullptr, int ldt = 0) const {
    if (is32) {
      f.store(dst, ld, dst_t, ldt);
    } else {
#pragma unroll
      for (int j = 0; j < PrefetchBf16<D, ROWS>::N; ++j) {
        const int idx = threadIdx.x + j * kThreads;
        if (idx >= ROWS * (D / 8)) continue;
        const int r = idx / (D / 8), c = (idx % (D / 8)) * 8;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if (dst) dst[r * ld + c + i] = (float)b.v[j][i];
          if (dst_t) dst_t[(c + i) * ldt + r] = (float)b.v[j][i];
        }
      }
    }
  }
};

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

// Write a 32 x 32 fp32 accumulator tile into LDS transposed (element (r, c) at [c * ld + r0 + r]) as
// a hi/lo pair of bf16 arrays.  Four consecutive rows go out as one 8-byte store.
__device__ __forceinline__ void acc_to_lds_t(const f32x16& acc, bf16* hi, bf16* lo, int ld, int r0) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    bf16x4 vh, vl;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bf16 a, b;
      split2(acc[4 * g + i], a, b);
      vh[i] = a;
      vl[i] = b;
    }
    const int e = acc_col() * ld + r0 + acc_row(4 * g);
    *(bf16x4*)(hi + e) = vh;
    *(bf16x4*)(lo + e) = vl;
  }
}

// Same for a 16 x 16 tile of mfma16 (element (r, c) at [c * ld + r0 + r]).
__device__ __forceinline__ void acc16_to_lds_t(const f32x4& acc, bf16* hi, bf16* lo, int ld, int r0) {
  bf16x4 vh, vl;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bf16 a, b;
    split2(acc[i], a, b);
    vh[i] = a;
    vl[i] = b;
  }
  const int e = (lane_id() & 15) * ld + r0 + 4 * (lane_id() >> 4);
  *(bf16x4*)(hi + e) = vh;
  *(bf16x4*)(lo + e) = vl;
}

// ---------------------------------------------------------------------------
// four-row patch prefetch: a thread holds rows 4 rg .. 4 rg + 3 of one column group, so a
// transposed copy goes out as 8-byte pieces of four consecutive rows.  Patch p of a thread:
// rg = p % 4 + 4 (p / (4 CG)), cg = (p / 4) % CG -- four consecutive lanes take four row groups of
// one column group, so an instruction reads whole rows.  Rows at or beyond nvalid read row 0 and
// are zeroed when stored.  ROWS must be a multiple of 16.
// ---------------------------------------------------------------------------
template <int D, int ROWS, int NTHR = kThreads>
struct PatchBf16 {
  static constexpr int RG = ROWS / 4, CG = D / 8, NP = RG * CG, N = (NP + NTHR - 1) / NTHR;
  bf16x8 v[N][4];
  __device__ __forceinline__ static void coords(int p, int& rg, int& cg) {
    rg = (p & 3) + 4 * (p / (4 * CG));
    cg = (p >> 2) % CG;
  }
  __device__ __forceinline__ void load(const bf16* g, long gstride, int nvalid, int lt) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      int rg, cg;
      coords(min(lt + j * NTHR, NP - 1), rg, cg);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * rg + i;
        v[j][i] = *(const bf16x8*)(g + (long)(r < nvalid ? r : 0) * gstride + 8 * cg);
      }
    }
  }
  // transposed copy: dst_t[c * ldt + r]
  __device__ __forceinline__ void store_t(bf16* dst_t, int ldt, int nvalid, int lt) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int p = lt + j * NTHR;
      if (NP % NTHR != 0 && p >= NP) continue;
      int rg, cg;
      coords(p, rg, cg);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        bf16x4 col;
#pragma unroll
        for (int i = 0; i < 4; ++i) col[i] = (4 * rg + i < nvalid) ? v[j][i][c] : (bf16)0.f;
        *(bf16x4*)(dst_t + (8 * cg + c) * ldt + 4 * rg) = col;
      }
    }
  }
  // row-major copy: dst[r * ld + c]
  __device__ __forceinline__ void store_rm(bf16* dst, int ld, int nvalid, int lt) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int p = lt + j * NTHR;
      if (NP % NTHR != 0 && p >= NP) continue;
      int rg, cg;
      coords(p, rg, cg);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bf16x8 x = v[j][i];
        if (4 * rg + i >= nvalid) x = bf16x8{};
        *(bf16x8*)(dst + (4 * rg + i) * ld + 8 * cg) = x;
      }
    }
  }
  // int16 rows of a block-floating-point tile: the scale of each of a patch's four rows (nvalid rows)
  __device__ __forceinline__ void load_scales(const float* scales, int nvalid, int lt, float (&sc)[N][4]) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      int rg, cg;
      coords(min(lt + j * NTHR, NP - 1), rg, cg);
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[j][i] = scales[4 * rg + i < nvalid ? 4 * rg + i : 0];
    }
  }
  // transposed copy of rowscale[i] x integer (the pieces hold int16 bit patterns), split into hi/lo
  // (exact: the value has at most 16 significant bits)
  __device__ __forceinline__ void store_t_s16(bf16* hi_t, bf16* lo_t, int ldt, const float (&rowscale)[N][4],
                                              int lt) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int p = lt + j * NTHR;
      if (NP % NTHR != 0 && p >= NP) continue;
      int rg, cg;
      coords(p, rg, cg);
      s16x8 x[4];  // whole pieces reinterpreted (a bit cast of one vector element reads element 0)
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = __builtin_bit_cast(s16x8, v[j][i]);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        bf16x4 ch, cl;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          bf16 a, b;
          split2(rowscale[j][i] * (float)x[i][c], a, b);
          ch[i] = a;
          cl[i] = b;
        }
        *(bf16x4*)(hi_t + (8 * cg + c) * ldt + 4 * rg) = ch;
        *(bf16x4*)(lo_t + (8 * cg + c) * ldt + 4 * rg) = cl;
      }
    }
  }
  // transposed copy of rowscale[i] x value, split into hi/lo
  __device__ __forceinline__ void store_t_scaled(bf16* hi_t, bf16* lo_t, int ldt, const float (&rowscale)[N][4],
                                                 int lt) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int p = lt + j * NTHR;
      if (NP % NTHR != 0 && p >= NP) continue;
      int rg, cg;
      coords(p, rg, cg);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        bf16x4 ch, cl;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          bf16 a, b;
          split2(rowscale[j][i] * (float)v[j][i][c], a, b);
          ch[i] = a;
          cl[i] = b;
        }
        *(bf16x4*)(hi_t + (8 * cg + c) * ldt + 4 * rg) = ch;
        *(bf16x4*)(lo_t + (8 * cg + c) * ldt + 4 * rg) = cl;
      }
    }
  }
};

// fp32 (or bf16) rows in four-row patches of 4 columns, stored transposed as a hi/lo bf16 pair.
template <int D, int ROWS, int NTHR = kThreads>
struct PatchF32 {
  static constexpr int RG = ROWS / 4, CG = D / 4, NP = RG * CG, N = (NP + NTHR - 1) / NTHR;
  f32x4 v[N][4];
  __device__ __forceinline__ static void coords(int p, int& rg, int& cg) {
    rg = (p & 3) + 4 * (p / (4 * CG));
    cg = (p >> 2) % CG;
  }
  __device__ __forceinline__ void load(const float* g32, const bf16* g16, long gstride, int nvalid, int lt) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      int rg, cg;
      coords(min(lt + j * NTHR, NP - 1), rg, cg);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * rg + i;
        const long e = (long)(r < nvalid ? r : 0) * gstride + 4 * cg;
        if (g32) {
          v[j][i] = *(const f32x4*)(g32 + e);
        } else {
          const bf16x4 b = *(const bf16x4*)(g16 + e);
#pragma unroll
          for (int k = 0; k < 4; ++k) v[j][i][k] = (float)b[k];
        }
      }
    }
  }
  // row-major hi/lo copy: hi[r * ld + c], lo[r * ld + c]
  __device__ __forceinline__ void store_rm(bf16* hi, bf16* lo, int ld, int nvalid, int lt) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int p = lt + j * NTHR;
      if (NP % NTHR != 0 && p >= NP) continue;
      int rg, cg;
      coords(p, rg, cg);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bf16x4 vh, vl;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          bf16 a, b;
          split2((4 * rg + i < nvalid) ? v[j][i][k] : 0.f, a, b);
          vh[k] = a;
          vl[k] = b;
        }
        *(bf16x4*)(hi + (4 * rg + i) * ld + 4 * cg) = vh;
        *(bf16x4*)(lo + (4 * rg + i) * ld + 4 * cg) = vl;
      }
    }
  }
  // row-major fp32 copy: dst[r * ld + c] (ld a multiple of 4)
  __device__ __forceinline__ void store_rm_f32(float* dst, int ld, int nvalid, int lt) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int p = lt + j * NTHR;
      if (NP % NTHR != 0 && p >= NP) continue;
      int rg, cg;
      coords(p, rg, cg);
#pragma unroll
      for (int i = 0; i < 4; ++i) *(f32x4*)(dst + (4 * rg + i) * ld + 4 * cg) = (4 * rg + i < nvalid) ? v[j][i] : f32x4{};
    }
  }
  __device__ __forceinline__ void store_t(bf16* hi_t, bf16* lo_t, int ldt, int nvalid, int lt) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int p = lt + j * NTHR;
      if (NP % NTHR != 0 && p >= NP) continue;
      int rg, cg;
      coords(p, rg, cg);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        bf16x4 ch, cl;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          bf16 a, b;
          split2((4 * rg + i < nvalid) ? v[j][i][c] : 0.f, a, b);
          ch[i] = a;
          cl[i] = b;
        }
        *(bf16x4*)(hi_t + (4 * cg + c) * ldt + 4 * rg) = ch;
        *(bf16x4*)(lo_t + (4 * cg + c) * ldt + 4 * rg) = cl;
      }
    }
  }
};

// fp32 rows (ROWS x D, contiguous D) stored row-major as a hi/lo bf16 pair (8-byte pieces).  Rows at
// or beyond nvalid read row 0 and are stored as zeros.
template <int D, int ROWS, int NTHR = kThreads>
struct PrefetchF32Split {
  static constexpr int VPR = D / 4, TOT = ROWS * VPR, N = (TOT + NTHR - 1) / NTHR;
  f32x4 v[N];
  __device__ __forceinline__ void load(const float* g, long gstride, int lt, int nvalid = ROWS) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = min(lt + j * NTHR, TOT - 1);
      const int r = idx / VPR;
      v[j] = *(const f32x4*)(g + (long)(r < nvalid ? r : 0) * gstride + (idx % VPR) * 4);
    }
  }
  __device__ __forceinline__ void store(bf16* hi, bf16* lo, int ld, int lt, int nvalid = ROWS) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = lt + j * NTHR;
      if (TOT % NTHR != 0 && idx >= TOT) continue;
      const int r = idx / VPR, c = (idx % VPR) * 4;
      bf16x4 vh, vl;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bf16 a, b;
        split2(r < nvalid ? v[j][i] : 0.f, a, b);
        vh[i] = a;
        vl[i] = b;
      }
      *(bf16x4*)(hi + r * ld + c) = vh;
      *(bf16x4*)(lo + r * ld + c) = vl;
    }
  }
};

// Marks a value loaded from HBM as settled: the empty asm consumes it (the load's wait is placed
// here) and yields a register value of its own.  Without it, a loop-carried value first loaded
// before a loop keeps the loop's wait analysis pessimistic: at the loop header the compiler merges
// the pending loads of the entry path with those of the back edge and waits for the shorter
// sequence's count in every pass.
template <typename T>
__device__ __forceinline__ void settle(T& x) {
  asm volatile("" : "+v"(x));
}

// Row-major register prefetch of a ROWS x D tile (bf16 or fp32) by NTHR threads: 16 consecutive
// lanes cover one 256-byte row segment, so the global loads are whole rows and the LDS writes are
// free of bank conflicts at any row pitch.  Rows at or beyond nvalid read row 0 and are stored as
// zeros; every load is issued unconditionally.
template <int D, int ROWS, int NTHR>
struct RowsBf16 {
  static constexpr int VPR = D / 8, TOT = ROWS * VPR, N = (TOT + NTHR - 1) / NTHR;
  bf16x8 v[N];
  __device__ __forceinline__ void load(const bf16* g, long gstride, int nvalid, int lt) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = min(lt + j * NTHR, TOT - 1), r = idx / VPR;
      v[j] = *gmem((const bf16x8*)(g + (long)(r < nvalid ? r : 0) * gstride + (idx % VPR) * 8));
    }
  }
  __device__ __forceinline__ void store(bf16* dst, int ld, int nvalid, int lt) const {
    if (nvalid >= ROWS) {  // whole tiles: no zero fill
#pragma unroll
      for (int j = 0; j < N; ++j) {
        const int idx = lt + j * NTHR;
        if (TOT % NTHR != 0 && idx >= TOT) continue;
        *(bf16x8*)(dst + (idx / VPR) * ld + (idx % VPR) * 8) = v[j];
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = lt + j * NTHR;
      if (TOT % NTHR != 0 && idx >= TOT) continue;
      const int r = idx / VPR;
      *(bf16x8*)(dst + r * ld + (idx % VPR) * 8) = r < nvalid ? v[j] : bf16x8{};
    }
  }
};

template <int D, int ROWS, int NTHR>
struct RowsF32 {
  static constexpr int VPR = D / 4, TOT = ROWS * VPR, N = (TOT + NTHR - 1) / NTHR;
  f32x4 v[N];
  __device__ __forceinline__ void load(const float* g, long gstride, int nvalid, int lt) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = min(lt + j * NTHR, TOT - 1), r = idx / VPR;
      v[j] = *gmem((const f32x4*)(g + (long)(r < nvalid ? r : 0) * gstride + (idx % VPR) * 4));
    }
  }
  // fp32 rows, or bf16 rows widened (g32 == nullptr)
  __device__ __forceinline__ void load(const float* g32, const bf16* g16, long gstride, int nvalid, int lt) {
    if (g32) {
      load(g32, gstride, nvalid, lt);
      return;
    }
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = min(lt + j * NTHR, TOT - 1), r = idx / VPR;
      const bf16x4 b = *gmem((const bf16x4*)(g16 + (long)(r < nvalid ? r : 0) * gstride + (idx % VPR) * 4));
#pragma unroll
      for (int i = 0; i < 4; ++i) v[j][i] = (float)b[i];
    }
  }
  __device__ __forceinline__ void store(float* dst, int ld, int nvalid, int lt) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = lt + j * NTHR;
      if (TOT % NTHR != 0 && idx >= TOT) continue;
      const int r = idx / VPR;
      *(f32x4*)(dst + r * ld + (idx % VPR) * 4) = r < nvalid ? v[j] : f32x4{};
    }
  }
  // row-major hi/lo bf16 pair (8-byte pieces)
  __device__ __forceinline__ void store_split(bf16* hi, bf16* lo, int ld, int nvalid, int lt) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = lt + j * NTHR;
      if (TOT % NTHR != 0 && idx >= TOT) continue;
      const int r = idx / VPR, e = r * ld + (idx % VPR) * 4;
      bf16x4 vh, vl;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bf16 x, y;
        split2(r < nvalid ? v[j][i] : 0.f, x, y);
        vh[i] = x;
        vl[i] = y;
      }
      *(bf16x4*)(hi + e) = vh;
      *(bf16x4*)(lo + e) = vl;
    }
  }
};

// ROWS x D int16 rows with an fp32 scale per row and 32-column block (row stride gstride elements,
// scale row stride sstride), staged through registers like RowsF32: 16-byte pieces of 8 values.
template <int D, int ROWS, int NTHR>
struct RowsQ16 {
  static constexpr int VPR = D / 8, TOT = ROWS * VPR, N = (TOT + NTHR - 1) / NTHR;
  static_assert(D % 32 == 0, "32-column scale blocks");
  s16x8 v[N];
  float sc[N];
  __device__ __forceinline__ void load(const short* g, const float* gs, long gstride, long sstride, int nvalid,
                                       int lt) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = min(lt + j * NTHR, TOT - 1), r = idx / VPR, p = idx % VPR;
      const long rr = r < nvalid ? r : 0;
      v[j] = *gmem((const s16x8*)(g + rr * gstride + p * 8));
      sc[j] = *gmem(gs + rr * sstride + p / 4);
    }
  }
  // row-major hi/lo bf16 pair of scale x value (16-byte pieces; exact: 16 significant bits)
  __device__ __forceinline__ void store_split(bf16* hi, bf16* lo, int ld, int nvalid, int lt) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = lt + j * NTHR;
      if (TOT % NTHR != 0 && idx >= TOT) continue;
      const int r = idx / VPR, e = r * ld + (idx % VPR) * 8;
      bf16x8 vh, vl;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        bf16 x, y;
        split2(r < nvalid ? sc[j] * (float)v[j][i] : 0.f, x, y);
        vh[i] = x;
        vl[i] = y;
      }
      *(bf16x8*)(hi + e) = vh;
      *(bf16x8*)(lo + e) = vl;
    }
  }
};

// Sum over the 2^log2n consecutive lanes that share a group (butterfly).
__device__ __forceinline__ float group_sum(float x, int n) {
  for (int m = 1; m < n; m <<= 1) x += __shfl_xor(x, m);
  return x;
}

// Value of another lane of the same 16-lane row by DPP.  Written as an update with a zero old value
// and bound_ctrl set (every control used here reads a valid lane, so neither takes effect) so that
// the move folds into the consuming add (v_add_f32_dpp).
template <int C>
__device__ __forceinline__ float dppf(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), C, 0xf, 0xf, true));
}

// Sum over the 16 lanes of a row (lanes 16 g .. 16 g + 15), every lane receives it: quad_perm
// [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror.
__device__ __forceinline__ float row16_sum(float x) {
  x += dppf<0xB1>(x);
  x += dppf<0x4E>(x);
  x += dppf<0x141>(x);
  x += dppf<0x140>(x);
  return x;
}

// DPP move with a row mask: rows outside RM (bit r = lanes 16 r .. 16 r + 15) receive 0.
template <int C, int RM>
__device__ __forceinline__ float dppf_rows(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), C, RM, 0xf, false));
}

// Inclusive prefix sum over the 64 lanes (lane l receives x_0 + ... + x_l): row_shr 1, 2, 4, 8 within
// each row of 16 lanes (lanes shifted in from outside the row read 0), then row_bcast:15 adds the
// last lane of rows 0 and 2 to rows 1 and 3, and row_bcast:31 adds lane 31 to rows 2 and 3.  Every
// lane must be active.
__device__ __forceinline__ float wave_scan_incl(float x) {
  x += dppf<0x111>(x);
  x += dppf<0x112>(x);
  x += dppf<0x114>(x);
  x += dppf<0x118>(x);
  x += dppf_rows<0x142, 0xA>(x);
  x += dppf_rows<0x143, 0xC>(x);
  return x;
}

// Value of lane `src` (a constant) of x, for every lane (v_readlane).
__device__ __forceinline__ float lane_value(float x, int src) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), src));
}

// Sum over the wavefront's 64 lanes, every lane receiving it: DPP within each row, then the four
// row sums.  Every lane must be active.
__device__ __forceinline__ float wave_total(float x) {
  x = row16_sum(x);
  return (lane_value(x, 0) + lane_value(x, 16)) + (lane_value(x, 32) + lane_value(x, 48));
}

}  // namespace ccq
