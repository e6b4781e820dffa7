// K3: leaf-block attention for every sampled (query, leaf block) pair, then
// the combine over samples.
//
// The reference gathers v[leaf] per sample and sums with the sample weights
// (_tree_mha.py:401-407; weighted_value_sum.cu:8-47).  With leaf blocks of LB
// keys each pair needs softmax(scale q K_blk^T) V_blk, so pairs are bucketed
// per leaf block (bucket.hip) and one workgroup per (leaf block, batch*head)
// keeps K_blk / V_blk in LDS while 64-pair tiles run through two MFMA
// products:  S^T = K Q^T (keys x queries), then O^T = V^T P^T with P^T taken
// straight from the S^T accumulator registers.  Each pair's w * o lands in
// its own slot of the partial buffer; combine_kernel sums the slots of each
// query in slot order, so the forward is deterministic without atomics.
// A launch covers the (batch, head)s bh0 .. bh0 + nbh - 1; the partial buffer
// holds the rows of those only, (nbh, L, S, D), so a caller with a bounded
// buffer runs the heads in groups (same kernels, same results).
#include "launch.h"

namespace ta {

struct LeafFwdArgs {
  int B, L, H, S, NL, LB, causal, coff, npiece, bh0, nbh;
  float scale_log2;
  const void *q, *k, *v;
  int64_t qsb, qsl, qsh, ksb, ksl, ksh, vsb, vsl, vsh;
  const int* order;
  const int* block_start;
  const int* piece_start;
  const int* piece_block;
  const float* slot_weight;
  void* partial;
};

template <typename E>
__device__ __forceinline__ void load8(E* o, const E* p) {
  if constexpr (sizeof(E) == 2) {
    *(uint4*)o = *(const uint4*)p;
  } else {
    *(float4*)o = *(const float4*)p;
    *(float4*)(o + 4) = *(const float4*)(p + 4);
  }
}

template <typename E, int D, int LBP>
__global__ __launch_bounds__(256) void leaf_fwd_kernel(LeafFwdArgs a) {
  using M = Mfma<E>;
  constexpr int KS = D + 8, VS = LBP + 8;  // padded LDS row strides
  extern __shared__ __align__(16) char smem[];
  E* Ks = (E*)smem;         // [LBP][KS]
  E* Vt = Ks + LBP * KS;    // [D][VS]

  int bh, beta;
  if (!group_bh_block(blockIdx.x, a.nbh, a.NL, bh, beta)) return;
  const int64_t prow0 = (int64_t)bh * a.L;  // partial rows of this (batch, head): (prow0 + l) * S + u
  bh += a.bh0;
  const int bb = bh / a.H, h = bh - bb * a.H;
  const int* bs = a.block_start + (int64_t)bh * (a.NL + 1);
  const int start = bs[beta], end = bs[beta + 1];
  if (start >= end) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, col = lane & 15, g = lane >> 4;
  const int LB = a.LB, S = a.S;
  const int64_t LS = (int64_t)a.L * S;
  const E* q = (const E*)a.q;
  const E* k = (const E*)a.k;
  const E* v = (const E*)a.v;

  for (int e = tid; e < LBP * D / 8; e += 256) {
    const int key = e / (D / 8), c = (e - key * (D / 8)) * 8;
    alignas(16) E kv[8];
    alignas(16) E vv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) { kv[i] = (E)0.f; vv[i] = (E)0.f; }
    if (key < LB) {
      const int64_t tok = (int64_t)beta * LB + key;
      if (k) load8(kv, k + bb * a.ksb + tok * a.ksl + h * a.ksh + c);
      load8(vv, v + bb * a.vsb + tok * a.vsl + h * a.vsh + c);
    }
    load8(Ks + key * KS + c, kv);
#pragma unroll
    for (int i = 0; i < 8; ++i) Vt[(c + i) * VS + key] = vv[i];
  }
  __syncthreads();

  // Each wave walks its own 16-pair tiles (tile j of the bucket goes to wave
  // j % 4); no workgroup barrier inside the loop.  The next tile's pair ids
  // and query rows are loaded while the current tile computes.
  const int* ord = a.order + (int64_t)bh * LS;
  int t0 = start + 16 * w;
  int ent = t0 + col < end ? ord[t0 + col] : -1;
  RowFrags<E, D> qf;
  qf.load(ent >= 0 ? q + bb * a.qsb + (int64_t)(ent / S) * a.qsl + h * a.qsh : nullptr, g);
  for (; t0 < end; t0 += 64) {
    const int cur = ent;
    RowFrags<E, D> qc = qf;
    const int t1 = t0 + 64;
    ent = t1 + col < end ? ord[t1 + col] : -1;
    qf.load(ent >= 0 ? q + bb * a.qsb + (int64_t)(ent / S) * a.qsl + h * a.qsh : nullptr, g);

    const bool valid = cur >= 0;
    const int l = valid ? cur / S : 0, u = valid ? cur - l * S : 0;
    f32x4 sacc[LBP / 16];
#pragma unroll
    for (int mt = 0; mt < LBP / 16; ++mt) {
      sacc[mt] = zero4();
      const E* ap = Ks + (16 * mt + col) * KS + M::KPL * g;
#pragma unroll
      for (int ks = 0; ks < D / M::K; ++ks) sacc[mt] = M::mma(ld_frag(ap + ks * M::K), qc.f[ks], sacc[mt]);
    }
    // keys < kmax are visible to this query
    const int kmax = valid ? (a.causal ? min(LB, l + a.coff - beta * LB + 1) : LB) : 0;
    float mx = -__builtin_inff();
#pragma unroll
    for (int mt = 0; mt < LBP / 16; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = 16 * mt + 4 * g + r;
        const float s = key < kmax ? sacc[mt][r] * a.scale_log2 : -__builtin_inff();
        sacc[mt][r] = s;
        mx = fmaxf(mx, s);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    float sum = 0.f;
#pragma unroll
    for (int mt = 0; mt < LBP / 16; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = (16 * mt + 4 * g + r) < kmax ? exp2f(sacc[mt][r] - mx) : 0.f;
        sacc[mt][r] = p;
        sum += p;
      }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);

    const int64_t qh = ((int64_t)bb * a.L + l) * a.H + h;
    const float f = (valid && sum > 0.f) ? a.slot_weight[qh * S + u] / sum : 0.f;
    E* dst = (E*)a.partial + ((prow0 + l) * S + u) * D;
#pragma unroll
    for (int md = 0; md < D / 16; ++md) {
      f32x4 o = zero4();
      const E* vrow = Vt + (16 * md + col) * VS;
#pragma unroll
      for (int ks = 0; ks < LBP / M::K; ++ks) o = M::mma(ld_frag_perm(vrow, ks, g), acc_operand<E>(sacc, ks), o);
      if (valid) store4(dst + 16 * md + 4 * g, o, f);
    }
  }
}

// 16-bit inputs.  One workgroup (four waves) per piece of at most kPieceFwd
// pairs of one leaf block (bucket.hip), so the heavy low blocks of causal runs
// are spread over many workgroups.  The block's K rows (the A operand of
// S^T = K Q^T) stay in LDS, read with 16-byte loads per tile; every wave keeps
// V^T (the A operand of O^T = V^T P^T) in registers for the whole piece, read
// once from a row-major LDS copy with transposing reads whose head-dim order
// puts eight consecutive dims of a pair's output in one lane, so each output
// row leaves in 16-byte stores.  The piece's pair list sits in LDS and every
// wave loads the query rows of its next two 16-pair tiles while the current
// one computes.
template <typename E, int D, int LBP>
__global__ __launch_bounds__(256, 2) void leaf_fwd16_kernel(LeafFwdArgs a) {
  using M = Mfma<E>;
  using F = typename M::frag;
  constexpr int KS = D / M::K;      // k-steps of S^T over head dims
  constexpr int MT = LBP / 16;      // key tiles of S^T
  constexpr int KK = LBP / M::K;    // k-steps of O^T over keys
  constexpr int NP = D / 32;        // 32-dim output groups (two O^T tiles each)
  constexpr int VS = D + 16;        // padded LDS row stride (elements)
  extern __shared__ __align__(16) char smem[];
  int* ord_s = (int*)smem;                  // [kPieceFwd] (l << 6) | u
  E* Vs = (E*)(smem + kPieceFwd * 4);       // [LBP][VS]
  E* Ks = Vs + LBP * VS;                    // [LBP][VS]

  int bh, piece;
  if (!group_bh_block(blockIdx.x, a.nbh, a.npiece, bh, piece)) return;
  const int64_t prow0 = (int64_t)bh * a.L;  // partial rows of this (batch, head): (prow0 + l) * S + u
  bh += a.bh0;
  const int beta = a.piece_block[(int64_t)bh * a.npiece + piece];
  if (beta < 0) return;
  const int bb = bh / a.H, h = bh - bb * a.H;
  const int* bs = a.block_start + (int64_t)bh * (a.NL + 1);
  const int p0 = bs[beta] + (piece - a.piece_start[(int64_t)bh * (a.NL + 1) + beta]) * kPieceFwd;
  const int np = min(bs[beta + 1] - p0, kPieceFwd);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, col = lane & 15, g = lane >> 4;
  const int LB = a.LB, S = a.S;
  const E* q = (const E*)a.q;
  const E* k = (const E*)a.k;
  const E* v = (const E*)a.v;

  const int* ord = a.order + (int64_t)bh * a.L * S + p0;
  for (int i = tid; i < np; i += 256) {
    const int ent = ord[i];
    const int l = ent / S;
    ord_s[i] = (l << 6) | (ent - l * S);
  }
  for (int e = tid; e < LBP * D / 8; e += 256) {
    const int key = e / (D / 8), c = (e - key * (D / 8)) * 8;
    uint4 vv = make_uint4(0, 0, 0, 0), kv = make_uint4(0, 0, 0, 0);
    if (key < LB) {
      const int64_t tok = (int64_t)beta * LB + key;
      vv = *(const uint4*)(v + bb * a.vsb + tok * a.vsl + h * a.vsh + c);
      if (k) kv = *(const uint4*)(k + bb * a.ksb + tok * a.ksl + h * a.ksh + c);
    }
    *(uint4*)(Vs + key * VS + c) = vv;
    *(uint4*)(Ks + key * VS + c) = kv;
  }
  __syncthreads();
  // V^T fragments (dims x keys), dims permuted so each lane's outputs are
  // eight consecutive dims
  F vf[2 * NP][KK];
#pragma unroll
  for (int md = 0; md < 2 * NP; ++md)
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) vf[md][kk] = perm_dim_frag<E>(Vs, VS, md, kk, lane);

  const int ntile = (np + 15) >> 4;
  const int coff = a.coff - beta * LB;  // key j of the block is visible to query l iff j <= l + coff
  // Three-set ring of (query-row fragments, summed sample weight): a step
  // waits for its own set (loaded two steps earlier), then issues the loads
  // of the tile two steps ahead, so no wait in a step covers a load issued
  // in the same step.
  struct QSet {
    RowFrags<E, D> q;
    float w;
  };
  auto fetch = [&](int t, QSet& r) {
    const int i = 16 * t + col;
    const bool ok = t < ntile && i < np;
    const int ent = ok ? ord_s[i] : 0;
    const int l = ent >> 6, u = ent & 63;
    r.q.load(ok ? q + bb * a.qsb + (int64_t)l * a.qsl + h * a.qsh : nullptr, g);
    r.w = ok ? a.slot_weight[(((int64_t)bb * a.L + l) * a.H + h) * S + u] : 0.f;
  };
  QSet qb[3];
  fetch(w, qb[0]);
  fetch(w + 4, qb[1]);
  auto step = [&](int t, QSet& cs, QSet& nxt) {
    cs.q.pin();
    pin_value(cs.w);
    const RowFrags<E, D>& cur = cs.q;
    const int i = 16 * t + col;
    const bool valid = i < np;
    const int ent = valid ? ord_s[i] : 0;
    const int l = ent >> 6, u = ent & 63;
    fetch(t + 8, nxt);
    f32x4 sacc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      sacc[mt] = zero4();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        sacc[mt] = M::mma(ld_frag(Ks + (16 * mt + col) * VS + ks * M::K + M::KPL * g), cur.f[ks], sacc[mt]);
    }
    const int kmax = valid ? (a.causal ? min(LB, l + coff + 1) : LB) : 0;
    float mx = -__builtin_inff();
    if (__any(kmax < LBP)) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          sacc[mt][r] = (16 * mt + 4 * g + r) < kmax ? sacc[mt][r] * a.scale_log2 : -__builtin_inff();
    } else {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) sacc[mt] *= a.scale_log2;
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) mx = fmaxf(mx, fmaxf(fmaxf(sacc[mt][0], sacc[mt][1]), fmaxf(sacc[mt][2], sacc[mt][3])));
    mx = col_max(mx);
    if (mx == -__builtin_inff()) mx = 0.f;  // no visible key (padding lanes): all p = 0
    float sum = 0.f;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = __builtin_amdgcn_exp2f(sacc[mt][r] - mx);
        sacc[mt][r] = p;
        sum += p;
      }
    sum = col_sum(sum);
    const int64_t qh = ((int64_t)bb * a.L + l) * a.H + h;
    const float f = (valid && sum > 0.f) ? cs.w * __builtin_amdgcn_rcpf(sum) : 0.f;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) sacc[mt] *= f;
    F pf[KK];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) pf[kk] = acc_operand<E>(sacc, kk);
    E* dst = (E*)a.partial + ((prow0 + l) * S + u) * D + 8 * g;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      f32x4 o0 = zero4(), o1 = zero4();
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        o0 = M::mma(vf[2 * p][kk], pf[kk], o0);
        o1 = M::mma(vf[2 * p + 1][kk], pf[kk], o1);
      }
      if (valid) {
        typedef __attribute__((ext_vector_type(8))) E e8;
        e8 o;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          o[r] = (E)o0[r];
          o[4 + r] = (E)o1[r];
        }
        *(e8*)(dst + 32 * p) = o;
      }
    }
  };
  for (int t = w; t < ntile; t += 12) {
    step(t, qb[0], qb[2]);
    if (t + 4 >= ntile) break;
    step(t + 4, qb[1], qb[0]);
    if (t + 8 >= ntile) break;
    step(t + 8, qb[2], qb[1]);
  }
}

// out[b,l,h,:] = sum over the query's distinct leaf blocks of the partial rows,
// for the L * nbh queries of the launch's (batch, head) group, position-major
// (consecutive threads write consecutive heads of one position).  With out32
// (a chunk of a problem with many samples) the sum goes to the float
// (B, L, H, D) rows instead: written by the first chunk, added by later ones.
// With oe (16-bit, the path-row backward's dout . out) out is also copied to
// the contiguous (B, L, H, D) rows oe.
template <typename E, int D>
__global__ __launch_bounds__(256) void combine_kernel(const E* __restrict__ partial, const int* __restrict__ slot_count,
                                                      E* __restrict__ out, int L, int H, int S, int bh0, int nbh,
                                                      int64_t osb, int64_t osl, int64_t osh, float* __restrict__ out32,
                                                      int first, E* __restrict__ oe) {
  constexpr int TPQ = D / 8;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = gid / TPQ;
  if (row >= (int64_t)L * nbh) return;
  const int part = (int)(gid - row * TPQ);
  const int64_t l = row / nbh, bhl = row - l * nbh;
  const int64_t bh = bh0 + bhl, bb = bh / H, h = bh - bb * H;
  const int64_t qh = (bb * L + l) * H + h;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  sum_rows8(acc, partial + (bhl * L + l) * S * D + 8 * part, D, slot_count[qh]);
  if (out32) {
    acc8f(out32 + qh * D + 8 * part, acc, first);
    return;
  }
  E* o = out + bb * osb + l * osl + h * osh + 8 * part;
  if constexpr (sizeof(E) == 2) {
    typedef __attribute__((ext_vector_type(8))) E e8;
    e8 v;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (E)acc[i];
    *(e8*)o = v;
    if (oe) *(e8*)(oe + qh * D + 8 * part) = v;
  } else {
    *(float4*)o = make_float4(acc[0], acc[1], acc[2], acc[3]);
    *(float4*)(o + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
}

static int fwd_smem(int D, int LBP, int es) {
  return (LBP * (D + 8) + D * (LBP + 8)) * es;
}

template <typename E, int D, int LBP>
static int fwd_smem_t() {
  return fwd_smem(D, LBP, (int)sizeof(E));
}

static int fwd16_smem(int D, int LBP) {
  return kPieceFwd * 4 + 2 * LBP * (D + 16) * 2;
}

int leaf_fwd_smem(const Plan& P) {
  const int s = P.esize == 2 ? fwd16_smem((int)P.D, padded_keys(P.geo.LB))
                             : fwd_smem((int)P.D, padded_keys(P.geo.LB), P.esize);
  return s <= 160 * 1024 ? s : -1;
}

template <typename E, int D, int LBP>
static hipError_t leaf_fwd_impl(const Plan& P, const void* q, const void* k, const void* v, void* out, char* rec,
                                void* partial, int bh0, int nbh, hipStream_t st) {
  LeafFwdArgs a;
  a.B = (int)P.B;
  a.L = (int)P.L;
  a.H = (int)P.H;
  a.S = (int)P.S;
  a.NL = P.geo.NL;
  a.LB = P.geo.LB;
  a.causal = P.p.causal == TA_CAUSAL_EXACT;
  a.coff = (int)(P.N - P.L);
  a.scale_log2 = P.p.scale * 1.4426950408889634f;
  a.q = q;
  a.k = P.p.tree_mode == TA_TREE_NODEKEYS ? nullptr : k;
  a.v = v;
  a.qsb = P.p.q_strides[0]; a.qsl = P.p.q_strides[1]; a.qsh = P.p.q_strides[2];
  a.ksb = P.p.k_strides[0]; a.ksl = P.p.k_strides[1]; a.ksh = P.p.k_strides[2];
  a.vsb = P.p.v_strides[0]; a.vsl = P.p.v_strides[1]; a.vsh = P.p.v_strides[2];
  a.order = (const int*)(rec + P.rec.order);
  a.block_start = (const int*)(rec + P.rec.block_start);
  a.npiece = P.npiece;
  a.piece_start = (const int*)(rec + P.rec.piece_start);
  a.piece_block = (const int*)(rec + P.rec.piece_block);
  a.slot_weight = (const float*)(rec + P.rec.slot_weight);
  a.partial = partial;
  a.bh0 = bh0;
  a.nbh = nbh;
  if constexpr (sizeof(E) == 2) {
    const int smem = fwd16_smem(D, LBP);
    hipError_t e = hipFuncSetAttribute((const void*)leaf_fwd16_kernel<E, D, LBP>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, smem);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((leaf_fwd16_kernel<E, D, LBP>), dim3(group_grid(nbh, P.npiece)), dim3(256), smem, st, a);
  } else {
    const int smem = fwd_smem_t<E, D, LBP>();
    hipError_t e = hipFuncSetAttribute((const void*)leaf_fwd_kernel<E, D, LBP>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, smem);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((leaf_fwd_kernel<E, D, LBP>), dim3(group_grid(nbh, P.geo.NL)), dim3(256), smem, st, a);
  }
  const int64_t nrows = (int64_t)nbh * P.L;
  const int64_t nthr = nrows * (D / 8);
  // a chunk adds into the problem's float output; with path rows the record
  // keeps a copy of the output (the backward's dout . out)
  E* oe = !P.acc.out32 && P.path_rows ? (E*)(rec + P.rec.out_e) : nullptr;
  hipLaunchKernelGGL((combine_kernel<E, D>), dim3((unsigned)((nthr + 255) / 256)), dim3(256), 0, st,
                     (const E*)a.partial, (const int*)(rec + P.rec.slot_count), (E*)out, (int)P.L, (int)P.H,
                     (int)P.S, bh0, nbh, P.p.o_strides[0], P.p.o_strides[1], P.p.o_strides[2], P.acc.out32,
                     P.acc.first, oe);
  return hipGetLastError();
}

template <typename E, int D>
static hipError_t leaf_fwd_lb(const Plan& P, const void* q, const void* k, const void* v, void* out, char* rec,
                              void* partial, int bh0, int nbh, hipStream_t st) {
  switch (padded_keys(P.geo.LB)) {
    case 32: return leaf_fwd_impl<E, D, 32>(P, q, k, v, out, rec, partial, bh0, nbh, st);
    case 64: return leaf_fwd_impl<E, D, 64>(P, q, k, v, out, rec, partial, bh0, nbh, st);
    default: return leaf_fwd_impl<E, D, 128>(P, q, k, v, out, rec, partial, bh0, nbh, st);
  }
}

template <typename E>
static hipError_t leaf_fwd_d(const Plan& P, const void* q, const void* k, const void* v, void* out, char* rec,
                             void* partial, int bh0, int nbh, hipStream_t st) {
  switch (P.D) {
    case 32: return leaf_fwd_lb<E, 32>(P, q, k, v, out, rec, partial, bh0, nbh, st);
    case 64: return leaf_fwd_lb<E, 64>(P, q, k, v, out, rec, partial, bh0, nbh, st);
    case 96: return leaf_fwd_lb<E, 96>(P, q, k, v, out, rec, partial, bh0, nbh, st);
    default: return leaf_fwd_lb<E, 128>(P, q, k, v, out, rec, partial, bh0, nbh, st);
  }
}

hipError_t launch_leaf_fwd_group(const Plan& P, const void* q, const void* k, const void* v, void* out, char* rec,
                                 void* partial, int bh0, int nbh, hipStream_t st) {
  if (P.geo.LB == 1) return launch_gather_fwd(P, v, out, rec, bh0, nbh, st);
  switch (P.p.dtype) {
    case TA_F32: return leaf_fwd_d<float>(P, q, k, v, out, rec, partial, bh0, nbh, st);
    case TA_BF16: return leaf_fwd_d<bf16>(P, q, k, v, out, rec, partial, bh0, nbh, st);
    default: return leaf_fwd_d<f16>(P, q, k, v, out, rec, partial, bh0, nbh, st);
  }
}

hipError_t launch_leaf_fwd(const Plan& P, const void* q, const void* k, const void* v, void* out, char* rec, char* ws,
                           hipStream_t st) {
  return launch_leaf_fwd_group(P, q, k, v, out, rec, ws + P.fws.partial, 0, (int)P.BH, st);
}

}  // namespace ta
