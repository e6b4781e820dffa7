// Shared device/host definitions for the gfx950 tree-attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "treeattn_amd.h"

namespace ta {

typedef __bf16 bf16;
typedef _Float16 f16;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) _Float16 f16x4;
typedef __attribute__((ext_vector_type(4))) float f32x4;

constexpr int kMaxDepth = 24;     // b^T = NL leaf blocks; b >= 2 so T <= 24 covers NL <= 2^24
constexpr int kMaxSamples = 64;   // one wavefront lane per sample
constexpr int kQueryTile = 64;    // queries per workgroup in the tree kernels
constexpr int kSampleDenseCols = 1024;  // widest level the sampler evaluates as level tiles
constexpr int kTreeDenseCols = 1024;    // widest level the backward's dense G tiles cover
constexpr int kDetMaxLeaves = TA_DET_MAX_LEAVES;  // deterministic mode: leaves per row held in LDS

// Tree geometry.  Child summaries are stored level-major: level lam (1..T)
// holds b^lam rows starting at off[lam], padded with zero rows to a multiple
// of 32 so every MFMA tile and 16-byte load of a level stays inside it;
// off[T+1] = NS.  Node i at depth d (0 <= i < b^d) has children rows
// off[d+1] + b*i + j.
struct Geo {
  int b, lb, T, NL, LB, NS;  // lb = log2(b): branching is a power of two
  int off[kMaxDepth + 2];
  int pw[kMaxDepth + 1];  // pw[i] = b^i
};

// ---------------------------------------------------------------- values ---

__device__ __forceinline__ float tof(float x) { return x; }
__device__ __forceinline__ float tof(bf16 x) { return (float)x; }
__device__ __forceinline__ float tof(f16 x) { return (float)x; }

template <typename E> __device__ __forceinline__ E fromf(float x) { return (E)x; }

// ------------------------------------------------------------------ MFMA ---
// v_mfma_f32_16x16x32_{bf16,f16} / v_mfma_f32_16x16x4_f32.  Lane l supplies
// A[row = l%16][k = KPL*(l/16) + i] and B[k = KPL*(l/16) + i][col = l%16];
// the accumulator lane holds D[row = 4*(l/16) + r][col = l%16], r < 4.

template <typename E> struct Mfma;

template <> struct Mfma<bf16> {
  static constexpr int K = 32, KPL = 8;
  typedef bf16x8 frag;
  __device__ static __forceinline__ f32x4 mma(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <> struct Mfma<f16> {
  static constexpr int K = 32, KPL = 8;
  typedef f16x8 frag;
  __device__ static __forceinline__ f32x4 mma(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <> struct Mfma<float> {
  static constexpr int K = 4, KPL = 1;
  typedef float frag;
  __device__ static __forceinline__ f32x4 mma(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

// KPL contiguous elements (16-byte aligned for 16-bit types).
__device__ __forceinline__ bf16x8 ld_frag(const bf16* p) { return *(const bf16x8*)p; }
__device__ __forceinline__ f16x8 ld_frag(const f16* p) { return *(const f16x8*)p; }
__device__ __forceinline__ float ld_frag(const float* p) { return *p; }

// KPL elements at stride s.
__device__ __forceinline__ bf16x8 ld_frag_strided(const bf16* p, int s) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = p[i * s];
  return r;
}
__device__ __forceinline__ f16x8 ld_frag_strided(const f16* p, int s) {
  f16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = p[i * s];
  return r;
}
__device__ __forceinline__ float ld_frag_strided(const float* p, int) { return *p; }

// KPL float values converted to the MFMA element type.
template <typename E> __device__ __forceinline__ typename Mfma<E>::frag cvt_frag(const float* p, int s);
template <> __device__ __forceinline__ bf16x8 cvt_frag<bf16>(const float* p, int s) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (bf16)p[i * s];
  return r;
}
template <> __device__ __forceinline__ f16x8 cvt_frag<f16>(const float* p, int s) {
  f16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (f16)p[i * s];
  return r;
}
template <> __device__ __forceinline__ float cvt_frag<float>(const float* p, int) { return *p; }

// The accumulator of a (keys x queries) product used directly as the k-operand
// of a product that reduces over keys.  Lane (g = l/16) holds keys 4g+r of
// each 16-row tile, so k-step ks of a 16-bit MFMA takes tiles 2ks and 2ks+1:
// slot i < 4 -> key 32ks + 4g + i, slot i >= 4 -> key 32ks + 16 + 4g + (i-4);
// an f32 MFMA step ks takes key 16(ks/4) + 4g + ks%4.  perm_key() gives that
// key so the other operand can be read in the same order.
template <typename E> __device__ __forceinline__ int perm_key(int ks, int g, int i);
template <> __device__ __forceinline__ int perm_key<bf16>(int ks, int g, int i) {
  return 32 * ks + 16 * (i >> 2) + 4 * g + (i & 3);
}
template <> __device__ __forceinline__ int perm_key<f16>(int ks, int g, int i) {
  return 32 * ks + 16 * (i >> 2) + 4 * g + (i & 3);
}
template <> __device__ __forceinline__ int perm_key<float>(int ks, int g, int) {
  return 16 * (ks >> 2) + 4 * g + (ks & 3);
}

// Operand row whose keys are contiguous, read in perm_key order.
__device__ __forceinline__ bf16x8 ld_frag_perm(const bf16* row, int ks, int g) {
  bf16x4 a = *(const bf16x4*)(row + 32 * ks + 4 * g);
  bf16x4 b = *(const bf16x4*)(row + 32 * ks + 16 + 4 * g);
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) { r[i] = a[i]; r[i + 4] = b[i]; }
  return r;
}
__device__ __forceinline__ f16x8 ld_frag_perm(const f16* row, int ks, int g) {
  f16x4 a = *(const f16x4*)(row + 32 * ks + 4 * g);
  f16x4 b = *(const f16x4*)(row + 32 * ks + 16 + 4 * g);
  f16x8 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) { r[i] = a[i]; r[i + 4] = b[i]; }
  return r;
}
__device__ __forceinline__ float ld_frag_perm(const float* row, int ks, int g) {
  return row[16 * (ks >> 2) + 4 * g + (ks & 3)];
}
// Same order, keys strided by `s` elements.
template <typename E> __device__ __forceinline__ typename Mfma<E>::frag ld_frag_perm_strided(const E* base, int s, int ks, int g) {
  typename Mfma<E>::frag r;
  if constexpr (Mfma<E>::KPL == 1) {
    r = base[perm_key<E>(ks, g, 0) * s];
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = base[perm_key<E>(ks, g, i) * s];
  }
  return r;
}

// Accumulator tiles as the k-operand (keys), converted to E.
template <typename E, int NT>
__device__ __forceinline__ typename Mfma<E>::frag acc_operand(const f32x4 (&acc)[NT], int ks) {
  typename Mfma<E>::frag r;
  if constexpr (Mfma<E>::KPL == 1) {
    r = acc[ks >> 2][ks & 3];
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      r[i] = (E)acc[2 * ks][i];
      r[i + 4] = (E)acc[2 * ks + 1][i];
    }
  }
  return r;
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Eight consecutive elements (16-byte aligned) as floats.
template <typename E>
__device__ __forceinline__ void ld8f(float* o, const E* p) {
  if constexpr (sizeof(E) == 2) {
    typedef __attribute__((ext_vector_type(8))) E e8;
    const e8 v = *(const e8*)p;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (float)v[i];
  } else {
    const float4 x = *(const float4*)p, y = *(const float4*)(p + 4);
    o[0] = x.x; o[1] = x.y; o[2] = x.z; o[3] = x.w; o[4] = y.x; o[5] = y.y; o[6] = y.z; o[7] = y.w;
  }
}

// dst[0..8) = v (first) or dst + v: float rows summed over the sample chunks
// of a problem with many samples (16-byte aligned dst).
__device__ __forceinline__ void acc8f(float* dst, const float* v, int first) {
  float4 a = make_float4(v[0], v[1], v[2], v[3]), b = make_float4(v[4], v[5], v[6], v[7]);
  if (!first) {
    const float4 x = *(const float4*)dst, y = *(const float4*)(dst + 4);
    a.x += x.x; a.y += x.y; a.z += x.z; a.w += x.w;
    b.x += y.x; b.y += y.y; b.z += y.z; b.w += y.w;
  }
  *(float4*)dst = a;
  *(float4*)(dst + 4) = b;
}

// dst[0..4) = scale * v as E, one 8-byte (16-bit E) or 16-byte (float) store;
// dst must be aligned to 4 elements.
template <typename E>
__device__ __forceinline__ void store4(E* dst, f32x4 v, float scale) {
  if constexpr (sizeof(E) == 2) {
    typedef __attribute__((ext_vector_type(4))) E v4;
    v4 o;
#pragma unroll
    for (int r = 0; r < 4; ++r) o[r] = (E)(v[r] * scale);
    *(v4*)dst = o;
  } else {
    *(f32x4*)dst = v * scale;
  }
}

template <typename E> __device__ __forceinline__ typename Mfma<E>::frag zero_frag() {
  typename Mfma<E>::frag r;
  if constexpr (Mfma<E>::KPL == 1) {
    r = 0.f;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (E)0.f;
  }
  return r;
}

// A-operand fragments of one 16-row tile held in registers for the whole
// reduction dimension D: lane (row l%16, k-group l/16) of row `row` (NULL ->
// zeros, for rows past the end).
template <typename E, int D>
struct RowFrags {
  typename Mfma<E>::frag f[D / Mfma<E>::K];
  __device__ __forceinline__ void load(const E* row, int g) {
#pragma unroll
    for (int ks = 0; ks < D / Mfma<E>::K; ++ks)
      f[ks] = row ? ld_frag(row + ks * Mfma<E>::K + Mfma<E>::KPL * g) : zero_frag<E>();
  }
  // The compiler waits here for the loads of these fragments, and no memory
  // operation moves above this point.  A software pipeline calls it before
  // issuing the next tile's loads: vmcnt counts loads and stores alike, so a
  // wait placed after newer loads (with stores in between) waits for all of
  // them.
  __device__ __forceinline__ void pin() const {
#pragma unroll
    for (int ks = 0; ks < D / Mfma<E>::K; ++ks) asm volatile("" ::"v"(f[ks]) : "memory");
  }
};
__device__ __forceinline__ void pin_value(float x) { asm volatile("" ::"v"(x) : "memory"); }

// X[16w + i][c] = A_i . B_row(c) for columns c < ncols (row row0 + c of the
// row-major B matrix with row length D; tile columns past ncols read row
// `rowmax`, a valid row whose results are never used), into X with row
// stride xs.  With kLo the B rows are split hi + lo and both products
// accumulate (float-accurate logits from 16-bit MFMA).  The next column
// tile's B fragments are loaded while the current tile's MFMAs run.
template <typename E, int D, bool kLo>
__device__ __forceinline__ void mfma_rows(const RowFrags<E, D>& A, float* X, int xs, const E* hi, const E* lo,
                                          int64_t row0, int ncols, int64_t rowmax, int lane, int w) {
  using M = Mfma<E>;
  constexpr int KS = D / M::K;
  const int col = lane & 15, g = lane >> 4;
  const int ntiles = (ncols + 15) >> 4;
  typename M::frag bh[KS], bl[KS];
  auto load = [&](int nt, typename M::frag(&h)[KS], typename M::frag(&l)[KS]) {
    const int64_t rb = (nt * 16 + col < ncols ? row0 + nt * 16 + col : rowmax) * D + M::KPL * g;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      h[ks] = ld_frag(hi + rb + ks * M::K);
      if constexpr (kLo) l[ks] = ld_frag(lo + rb + ks * M::K);
    }
  };
  if (ntiles > 0) load(0, bh, bl);
  for (int nt = 0; nt < ntiles; ++nt) {
    typename M::frag nh[KS], nl[KS];
    if (nt + 1 < ntiles) load(nt + 1, nh, nl);
    f32x4 c = zero4();
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      c = M::mma(A.f[ks], bh[ks], c);
      if constexpr (kLo) c = M::mma(A.f[ks], bl[ks], c);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) X[(16 * w + 4 * g + r) * xs + nt * 16 + col] = c[r];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      bh[ks] = nh[ks];
      if constexpr (kLo) bl[ks] = nl[ks];
    }
  }
}

// acc[0..8) += sum_{u < n} rows[u*stride .. +8) (E values, 16-byte aligned
// when E is 16-bit), in u order.  16-bit rows are loaded sixteen at a time as
// raw 16-byte words (converted after the loads), float rows eight at a time,
// so that many loads are in flight per thread.
template <typename E>
__device__ __forceinline__ void sum_rows8(float* acc, const E* rows, int64_t stride, int n) {
  if constexpr (sizeof(E) == 2) {
    for (int u0 = 0; u0 < n; u0 += 16) {
      uint4 x[16];
#pragma unroll
      for (int j = 0; j < 16; ++j)
        x[j] = u0 + j < n ? *(const uint4*)(rows + (int64_t)(u0 + j) * stride) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        typedef __attribute__((ext_vector_type(8))) E v8;
        const v8 v = __builtin_bit_cast(v8, x[j]);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] += (float)v[i];
      }
    }
  } else {
    for (int u0 = 0; u0 < n; u0 += 8) {
      float4 x[8][2];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float* p = (const float*)rows + (int64_t)(u0 + j) * stride;
        x[j][0] = u0 + j < n ? *(const float4*)p : make_float4(0, 0, 0, 0);
        x[j][1] = u0 + j < n ? *(const float4*)(p + 4) : make_float4(0, 0, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        acc[0] += x[j][0].x; acc[1] += x[j][0].y; acc[2] += x[j][0].z; acc[3] += x[j][0].w;
        acc[4] += x[j][1].x; acc[5] += x[j][1].y; acc[6] += x[j][1].z; acc[7] += x[j][1].w;
      }
    }
  }
}

// ------------------------------------------------ transposing LDS reads ---
typedef __attribute__((ext_vector_type(4))) short s16x4;
typedef __attribute__((ext_vector_type(8))) short s16x8;

// Four 16-bit values through ds_read_b64_tr_b16, gfx950's transposing LDS
// read of a row-major tile X (row stride rs elements): within each group of
// 16 lanes, lane i receives element i%4 of the 8-byte slots that lanes
// 4r + i/4 (r = 0..3) point at.  Lane j of a group points at row k0 + j/4 and
// an 8-byte-aligned column c(j%4) of its choice, so lane i gets
// X[k0 + r][c(i/4) + i%4], r = 0..3.
template <typename E>
__device__ __forceinline__ s16x4 tr_read4(const E* X, int rs, int row, int col) {
  typedef __attribute__((address_space(3))) s16x4* lp;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lp)(X + row * rs + col));
}

// An MFMA operand fragment of k = 8 values from the row-major [k][n] LDS tile
// X (row stride rs): rows k0a..k0a+3 then k0b..k0b+3 of column n0 + lane % 16,
// through two transposing reads.
template <typename E>
__device__ __forceinline__ typename Mfma<E>::frag tr_frag(const E* X, int rs, int k0a, int k0b, int n0, int lane) {
  const int j = lane & 15;
  const s16x4 lo = tr_read4(X, rs, k0a + (j >> 2), n0 + 4 * (j & 3));
  const s16x4 hi = tr_read4(X, rs, k0b + (j >> 2), n0 + 4 * (j & 3));
  const s16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(typename Mfma<E>::frag, v);
}

// A-operand fragment of a (head dims x keys) product read from the row-major
// [key][dim] LDS tile X: tile md = 2p + e, row m <-> dim 32p + 8(m/4) + 4e +
// m%4 (so that the product's output gives each lane eight consecutive dims),
// keys in the order of acc_operand for k-step kk (32kk + 4g + i, then
// 32kk + 16 + 4g + i).
template <typename E>
__device__ __forceinline__ typename Mfma<E>::frag perm_dim_frag(const E* X, int rs, int md, int kk, int lane) {
  const int j = lane & 15, g = lane >> 4;
  const int cc = 32 * (md >> 1) + 8 * (j & 3) + 4 * (md & 1);
  const s16x4 lo = tr_read4(X, rs, 32 * kk + 4 * g + (j >> 2), cc);
  const s16x4 hi = tr_read4(X, rs, 32 * kk + 16 + 4 * g + (j >> 2), cc);
  const s16x8 x = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(typename Mfma<E>::frag, x);
}

// ------------------------------------------------------- XCD placement ---
// Workgroups are dispatched to the 8 XCDs of the chip round-robin by linear
// id, and each XCD has its own L2.  xcd_bh_block maps linear id i to
// (bh, beta) so that every leaf block of one (batch, head) runs on the same
// XCD, in ascending beta (the heavy low blocks of causal runs first): the
// rows that the blocks' pairs gather (queries, output gradients) then stay
// in that XCD's L2.  Launch xcd_grid(nbh, nl) workgroups; ids with no work
// get false.
constexpr int kXcds = 8;
__device__ __forceinline__ bool xcd_bh_block(int i, int nbh, int nl, int& bh, int& beta) {
  const int x = i % kXcds, j = i / kXcds;
  const int r = j / nl;
  beta = j - r * nl;
  bh = r * kXcds + x;
  return bh < nbh;
}
inline unsigned xcd_grid(int64_t nbh, int nl) {
  return (unsigned)(((nbh + kXcds - 1) / kXcds) * kXcds * nl);
}
// A launch over a group of nbh (batch, head)s: with at least one per XCD the
// mapping above; with fewer, each (batch, head)'s blocks are spread over all
// XCDs in order (linear id = bh * nl + beta), so no XCD idles.  Launch
// group_grid(nbh, nl) workgroups.
__device__ __forceinline__ bool group_bh_block(int i, int nbh, int nl, int& bh, int& beta) {
  if (nbh >= kXcds) return xcd_bh_block(i, nbh, nl, bh, beta);
  bh = i / nl;
  beta = i - bh * nl;
  return bh < nbh;
}
inline unsigned group_grid(int64_t nbh, int nl) {
  return nbh >= kXcds ? xcd_grid(nbh, nl) : (unsigned)(nbh * nl);
}

// ------------------------------------------------------- DPP exchanges ---
// x from lane (i - R) mod 16 of the same 16-lane row (DPP row_ror).
template <int R>
__device__ __forceinline__ float dpp_row_ror(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x120 + R, 0xf, 0xf, false));
}
// x from lane j ^ M of this 16-lane row (M = 1, 2, 4, 8; j = lane & 15), by
// DPP moves: quad_perm [1, 0, 3, 2] for M = 1, [2, 3, 0, 1] for M = 2, a
// rotation by 8 for M = 8, and for M = 4 the rotation by 4 or by 12, whichever
// lands on j ^ 4.  No LDS traffic, unlike a shuffle.
template <int M>
__device__ __forceinline__ float row_xor(float x, int j) {
  if constexpr (M == 1) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xf, 0xf, false));
  } else if constexpr (M == 2) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xf, 0xf, false));
  } else if constexpr (M == 8) {
    return dpp_row_ror<8>(x);
  } else {
    const float dn = dpp_row_ror<M>(x), up = dpp_row_ror<16 - M>(x);
    return (j & M) ? dn : up;
  }
}

// ------------------------------------------------------ vector-ALU dots ---

__device__ __forceinline__ float logsig(float x) { return fminf(x, 0.f) - log1pf(expf(-fabsf(x))); }

// q . c for one query row (E) and one float summary row, D a multiple of 8
template <typename E>
__device__ __forceinline__ float dot_row(const E* q, const float* c, int D) {
  float acc = 0.f;
  for (int i = 0; i < D; i += 8) {
    float x[8];
    if constexpr (sizeof(E) == 2) {
      typedef __attribute__((ext_vector_type(8))) E v8;
      const v8 v = *(const v8*)(q + i);
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = (float)v[j];
    } else {
      const float4 a = *(const float4*)(q + i), b = *(const float4*)(q + i + 4);
      x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    }
    const float4 c0 = *(const float4*)(c + i), c1 = *(const float4*)(c + i + 4);
    acc += x[0] * c0.x + x[1] * c0.y + x[2] * c0.z + x[3] * c0.w + x[4] * c1.x + x[5] * c1.y + x[6] * c1.z +
           x[7] * c1.w;
  }
  return acc;
}

// ------------------------------------------------------------ reductions ---

// x op x[lane ^ 16] and x op x[lane ^ 32] through gfx950's v_permlane16_swap
// and v_permlane32_swap (VALU lane swaps, no LDS round trip).  With both
// registers holding x, the swap leaves (x[i & ~16], x[i | 16]) (resp. 32) in
// lane i, whose op is the xor-partner reduction.  The swap is issued as inline
// asm with both registers as in/out operands: the compiler's own lowering of
// the two-result builtin has been seen to reuse the first result for both.
// The s_nops cover the VALU-write -> permlane-read and permlane -> VALU-read
// distances.
__device__ __forceinline__ void swap16(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap32(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ float xor16_sum(float x) {
  float a = x, b = x;
  swap16(a, b);
  return a + b;
}
__device__ __forceinline__ float xor32_sum(float x) {
  float a = x, b = x;
  swap32(a, b);
  return a + b;
}
__device__ __forceinline__ float xor16_max(float x) {
  float a = x, b = x;
  swap16(a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float xor32_max(float x) {
  float a = x, b = x;
  swap32(a, b);
  return fmaxf(a, b);
}
// Sum / max over the four lanes col, col+16, col+32, col+48 (the lane groups
// of an MFMA accumulator column).
__device__ __forceinline__ float col_sum(float x) { return xor32_sum(xor16_sum(x)); }
__device__ __forceinline__ float col_max(float x) { return xor32_max(xor16_max(x)); }

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}

// -------------------------------------------------------------- counter RNG ---
// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11).  Uniform i of a tensor is
// word i%4 of philox(ctr = (lo(i/4), hi(i/4), 0, 0), key = seed), mapped to
// ((x >> 9) + 0.5) * 2^-23, exact in float32 and inside [2^-24, 1 - 2^-24].

struct Philox4 { uint32_t w[4]; };

__device__ __host__ inline Philox4 philox4x32_10(uint64_t ctr, uint64_t seed) {
  uint32_t c0 = (uint32_t)ctr, c1 = (uint32_t)(ctr >> 32), c2 = 0, c3 = 0;
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r > 0) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
    uint64_t p0 = (uint64_t)0xD2511F53u * c0;
    uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
    uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
  }
  Philox4 o;
  o.w[0] = c0; o.w[1] = c1; o.w[2] = c2; o.w[3] = c3;
  return o;
}

// Packed path bits (bit p = p-th root-to-leaf bit, bytes least-significant
// bit first) <-> leaf block id (those bits most-significant first), nbits in
// [1, 31]: one bit reversal of the little-endian word.
__device__ __forceinline__ uint32_t path_leaf(const uint8_t* p, int nbits, int nbytes) {
  uint32_t w = 0;
  for (int k = 0; k < nbytes; ++k) w |= (uint32_t)p[k] << (8 * k);
  return nbits > 0 ? __builtin_bitreverse32(w) >> (32 - nbits) : 0u;
}
__device__ __forceinline__ uint32_t leaf_path_word(uint32_t id, int nbits) {
  return nbits > 0 ? __builtin_bitreverse32(id << (32 - nbits)) : 0u;
}

__device__ __host__ inline float word_to_uniform(uint32_t x) {
  return ((float)(x >> 9) + 0.5f) * (1.0f / 8388608.0f);
}

// ---------------------------------------------------------- record layout ---
// Byte offsets of the saved record and the workspaces inside the caller's
// buffers (256-byte aligned pieces).

struct RecordLayout {
  int64_t summaries;   // float (BH, NS, D)
  int64_t sum_hi;      // E (BH, NS, D): E-rounded summaries (float inputs: unused)
  int64_t sum_lo;      // E (BH, NS, D): summaries - hi
  int64_t sum_t;       // E (BH, D, NS): hi, transposed (float inputs: float)
  int64_t means;       // float (BH, NL, D) leaf-block means
  int64_t segs;        // float: sums of 64 and of 64^2 consecutive means (NL >= 128)
  int64_t leaf;        // int (B, L, H, S): leaf block of each sample
  int64_t slot_leaf;   // int (B, L, H, S): distinct leaf blocks, ascending
  int64_t slot_weight; // float (B, L, H, S): summed weight per distinct leaf block
  int64_t slot_count;  // int (B, L, H)
  int64_t lse;         // float (B, L, H): log of the summed exp(log-prob) over the query's samples
  int64_t hist;        // int (BH, NL, nchunk): pair counts, then scanned offsets
  int64_t block_start; // int (BH, NL + 1)
  int64_t order;       // int (BH, L*S): (l*S + u) grouped by leaf block
  int64_t piece_start; // int (BH, NL + 1): first leaf-forward piece of each block, exclusive scan
  int64_t piece_block; // int (BH, npiece): leaf block of each piece, -1 past the last
  int64_t seg_sum;     // int (BH, nseg): bucket counts per histogram scan segment
  int64_t dstar;       // int (L): reference causal mode: first uncorrected depth per query
  int64_t logA;        // float (B, L, H, T + 1): exact causal with sparse levels, boundary log-masses
  int64_t sort_keys;   // uint32 (2, B, L, H, S): bucketing by sort, key double buffer
  int64_t sort_vals;   // int (2, B, L, H, S): bucketing by sort, value double buffer
  int64_t sort_hist;   // int (256, tiles of 2048 keys + 1): the sort's per-tile digit counts, digit totals
  int64_t out_e;       // E (B, L, H, D): a copy of the forward output (path rows, one chunk)
  int64_t total;
};

struct FwdWorkspaceLayout {
  int64_t partial;  // E (BH, L, S, D): w * o per distinct leaf block
  int64_t total;
};

struct BwdWorkspaceLayout {
  int64_t delta;     // float (B, L, H, S): dout . o per distinct leaf block
  int64_t dq_part;   // E (B, L, H, S, D): leaf dq per distinct leaf block
  int64_t dlogp;     // float (B, L, H, S): gradient of each distinct leaf block's summed log-prob
  int64_t dk_leaf;   // float (B, N, H, D)
  int64_t gt;        // E (BH, Lp/64, NS, 64): gradient of the child logits, transposed per 64-query tile
  int64_t qt;        // E (BH, Lp/64, D, 64): queries transposed per 64-query tile
  int64_t dsum_part; // float (qsplit, BH, NS, D)
  int64_t dsum;      // float (BH, NS, D)
  int64_t rc_coef;   // float (B, L, H, T): reference causal mode, boundary-mass gradient scale
  int64_t rc_rho;    // float (B, L, H, T): reference causal mode, on-path share of each boundary mass
  int64_t rc_g;      // float (B, L, H, T): reference causal mode, boundary children's gradient (band depths)
  int64_t mean;      // float (B, L, H): path rows, dout . out over the query's samples
  int64_t dcp;       // float (BH, NL, T*b, D): path rows, each leaf block's gradient of its path's children
  int64_t total;
};

constexpr int kQueryChunk = 256; // queries per bucketing chunk (one wavefront each)
constexpr int kBucketWin = 2048; // leaf blocks the counting sort's LDS window holds; more sort by keys
// A leaf block's pairs are cut into pieces of at most kPieceFwd pairs, one
// leaf-forward workgroup each, so the heavy low blocks of causal runs (a
// block near the start is reachable from every later query) do not leave
// one workgroup running long after the others.
constexpr int kPieceFwd = 1024;

}  // namespace ta
