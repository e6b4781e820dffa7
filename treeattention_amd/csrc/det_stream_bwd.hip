// Streaming backward of the deterministic mode for 16-bit inputs (the
// gradient of det_stream_fwd_kernel's function, _tree_mha.py:271-321),
// without any (L, N) buffer.
//
// Per query q and leaf n: W = exp(lp) (non-causal) or exp(lp - lse_q) on
// n <= q (causal); dW = dout_q . v_n; dlp = W (dW - delta_q) with
// delta_q = dout_q . out_q (causal) or 0; for a node with logit x and
// children sums A_L, A_R of dlp, G = sigmoid(-x) A_L - sigmoid(x) A_R;
// dq = sum G k_node, dk_node = sum_q G q, dv_n = sum_q W dout_q.
//
// The N leaves split into 64-leaf chunks (subtrees at depth tt = T - 6).  A
// chunk's 63 internal nodes get G from the chunk's own leaves; the tt levels
// above see the chunk only through its total A_r(q) = sum of dlp over its
// leaves, so they are the same computation on a coarse tree of NC = 2^tt
// leaves (done by the caller with ta_det_grad and two products).  One routine
// (tile_grad) does a (64-query tile, chunk) pair:
//   node logits X^T by MFMA (as the forward), leaf log-weights by a register
//   expansion (4 threads per query, 16 leaves each), W; dW^T = V dout^T by
//   MFMA into the logit tile (the logits are in registers by then); dlp;
//   bottom-up sums inside each thread's 16 leaves, then across the 4 threads
//   by lane shuffles; G of the 63 nodes into an LDS tile (input type).
// det_bwd_q_kernel (one workgroup per 64 queries) walks the chunks: dq_sub +=
//   G K_sub (MFMA, K^T via transposing LDS reads) and the chunk totals.
// det_bwd_kv_kernel (one workgroup per chunk) walks the query tiles:
//   dv += W^T dout and dk_sub += G^T q (MFMA, all operands through
//   transposing LDS reads).
// Every output element has one writer; no atomics.
#include "launch.h"

namespace ta {

constexpr int kDbQ = 64;       // queries per tile
constexpr int kDbLeaves = 64;  // leaves per chunk
constexpr int kDbCols = 80;    // node columns per chunk: <= 9 ancestors + 63 subtree nodes, padded

__device__ __forceinline__ float db_logsig(float x) {
  const float e = __builtin_amdgcn_exp2f(-fabsf(x) * 1.4426950408889634f);
  return fminf(x, 0.f) - 0.69314718055994531f * __builtin_amdgcn_logf(1.f + e);
}
__device__ __forceinline__ float db_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
// G = sigmoid(-x) A_L - sigmoid(x) A_R, with sigmoid(+-|x|) from one exp
__device__ __forceinline__ float node_grad(float x, float al, float ar) {
  const float e = __builtin_amdgcn_exp2f(-fabsf(x) * 1.4426950408889634f);
  const float sp = __builtin_amdgcn_rcpf(1.f + e), sn = e * sp;  // sigmoid(|x|), sigmoid(-|x|)
  const float s = x >= 0.f ? sp : sn, s_neg = x >= 0.f ? sn : sp;
  return s_neg * al - s * ar;
}

struct DetBwdArgs {
  const void* q;
  int64_t qsb, qsl, qsh;
  const void* g;  // output gradient
  int64_t gsb, gsl, gsh;
  const void* kn;  // heap-ordered node keys (input type), (batch, node, head) strides
  int64_t ksb, ksn, ksh;
  const void* v;
  int64_t vsb, vsl, vsh;
  const float* lse;    // (B, H, L) causal
  const float* delta;  // (B, H, L) causal
  float* dq;           // (B, H, L, D) subtree part of dq
  float* achunk;       // (B, H, L, NC) chunk totals of dlp
  float* dkn;          // (N-1, B, H, D) node-key gradients (subtree rows)
  void* dv;
  int64_t dvsb, dvsl, dvsh;
  int B, L, H, T, causal;
};

// Heap index of column cix of chunk r (ancestors first, then the subtree's
// nodes breadth-first), or -1 for padding.
__device__ __forceinline__ int chunk_node(int cix, int r, int tt) {
  if (cix < tt) return (1 << cix) - 1 + (r >> (tt - cix));
  if (cix < tt + kDbLeaves - 1) {
    const int m = cix - tt, dep = 31 - __builtin_clz(m + 1);
    return (1 << (tt + dep)) - 1 + (r << dep) + (m + 1 - (1 << dep));
  }
  return -1;
}

// Row padding of 8 elements keeps the chunk-major kernel at D <= 64 within
// 80 KiB of LDS (two workgroups per CU).
template <typename E, int D>
struct DbTiles {
  static constexpr int RS = D + 8;           // row stride (elements) of K / V / q / dout tiles
  static constexpr int XS = kDbCols + 4;     // float row stride of the logit (then dW) tile
  static constexpr int PS = kDbLeaves + 8;   // row stride (elements) of the W / G tiles
};

// Stage chunk r's node-key columns and value rows into Ks / Vs (all threads).
template <typename E, int D>
__device__ __forceinline__ void stage_chunk(const DetBwdArgs& a, int bb, int h, int r, int tt, E* Ks, E* Vs,
                                            int tid) {
  constexpr int RS = DbTiles<E, D>::RS;
  const E* kn = (const E*)a.kn;
  const E* v = (const E*)a.v;
  constexpr int NKL = (kDbCols * (D / 8) + 255) / 256, NVL = (kDbLeaves * (D / 8) + 255) / 256;
  uint4 kr[NKL], vr[NVL];
#pragma unroll
  for (int j = 0; j < NKL; ++j) {
    const int e = tid + 256 * j, cix = e / (D / 8), d0 = (e - cix * (D / 8)) * 8;
    const int node = e < kDbCols * (D / 8) ? chunk_node(cix, r, tt) : -1;
    kr[j] = node >= 0 ? *(const uint4*)(kn + bb * a.ksb + (int64_t)node * a.ksn + h * a.ksh + d0)
                      : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < NVL; ++j) {
    const int e = tid + 256 * j, lf = e / (D / 8), d0 = (e - lf * (D / 8)) * 8;
    const int64_t tok = (int64_t)r * kDbLeaves + lf;
    vr[j] = e < kDbLeaves * (D / 8) ? *(const uint4*)(v + bb * a.vsb + tok * a.vsl + h * a.vsh + d0)
                                     : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < NKL; ++j) {
    const int e = tid + 256 * j;
    if (e < kDbCols * (D / 8)) *(uint4*)(Ks + (e / (D / 8)) * RS + (e % (D / 8)) * 8) = kr[j];
  }
#pragma unroll
  for (int j = 0; j < NVL; ++j) {
    const int e = tid + 256 * j;
    if (e < kDbLeaves * (D / 8)) *(uint4*)(Vs + (e / (D / 8)) * RS + (e % (D / 8)) * 8) = vr[j];
  }
}

// One (query tile, chunk) pair.  Wave w owns tile queries 16w..16w+15 (qa /
// ga: their q and dout rows as MFMA fragments); thread t handles query t/4,
// leaves 16 (t%4) .. +15.  Writes G (subtree node m at column m; column 63
// stays zero) and, when Ws is given, W into rows of this wave's queries.
// Returns the chunk total of dlp for the thread's query.  Xs rows are this
// wave's only, so no workgroup barrier is needed inside.
template <typename E, int D>
__device__ __forceinline__ float tile_grad(const RowFrags<E, D>& qa, const RowFrags<E, D>& ga, const E* Ks,
                                           const E* Vs, float* Xs, E* Gs, E* Ws, int r, int tt, int lq, float lse_q,
                                           float delta_q, int causal, int tid) {
  using M = Mfma<E>;
  using TL = DbTiles<E, D>;
  constexpr int RS = TL::RS, XS = TL::XS, PS = TL::PS, KS = D / M::K;
  const int lane = tid & 63, w = tid >> 6, col = lane & 15, g = lane >> 4;
  const int qi = tid >> 2, jq = tid & 3;
  const int nct = (tt + kDbLeaves - 1 + 15) >> 4;
  for (int ct = 0; ct < nct; ++ct) {
    f32x4 x = zero4();
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) x = M::mma(ld_frag(Ks + (16 * ct + col) * RS + ks * M::K + M::KPL * g), qa.f[ks], x);
    *(f32x4*)(Xs + (16 * w + col) * XS + 16 * ct + 4 * g) = x;
  }
  const float* xr = Xs + qi * XS;
  // logits this thread needs: the two shared subtree decisions and its 15 nodes
  const float x0 = xr[tt], x1 = xr[tt + 1 + (jq >> 1)];
  float xg[15];
#pragma unroll
  for (int e = 0; e < 4; ++e)
#pragma unroll
    for (int i = 0; i < (1 << e); ++i) xg[(1 << e) - 1 + i] = xr[tt + (1 << (2 + e)) - 1 + (jq << e) + i];
  float pre = 0.f;
  for (int d = 0; d < tt; ++d) {
    const float x = xr[d], ls = db_logsig(x);
    pre += ((r >> (tt - 1 - d)) & 1) ? ls - x : ls;
  }
  {
    const float l0s = db_logsig(x0), l1s = db_logsig(x1);
    pre += (jq >> 1) ? l0s - x0 : l0s;
    pre += (jq & 1) ? l1s - x1 : l1s;
  }
  float av[16];
  av[0] = pre;
#pragma unroll
  for (int e = 0; e < 4; ++e)
#pragma unroll
    for (int i = (1 << e) - 1; i >= 0; --i) {
      const float x = xg[(1 << e) - 1 + i], ls = db_logsig(x);
      av[2 * i + 1] = av[i] + ls - x;
      av[2 * i] = av[i] + ls;
    }
  const int nb = r * kDbLeaves + 16 * jq;
#pragma unroll
  for (int i = 0; i < 16; ++i)
    av[i] = causal ? (nb + i <= lq ? db_exp(av[i] - lse_q) : 0.f) : db_exp(av[i]);  // W
  if (Ws) {
    typedef __attribute__((ext_vector_type(8))) E e8;
    e8 p0, p1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      p0[i] = (E)av[i];
      p1[i] = (E)av[8 + i];
    }
    *(e8*)(Ws + qi * PS + 16 * jq) = p0;
    *(e8*)(Ws + qi * PS + 16 * jq + 8) = p1;
  }
  // dW^T = V dout^T over the logit tile (this wave's rows; its logits are in registers)
#pragma unroll
  for (int ct = 0; ct < kDbLeaves / 16; ++ct) {
    f32x4 d = zero4();
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) d = M::mma(ld_frag(Vs + (16 * ct + col) * RS + ks * M::K + M::KPL * g), ga.f[ks], d);
    *(f32x4*)(Xs + (16 * w + col) * XS + 16 * ct + 4 * g) = d;
  }
  float dl[16];
#pragma unroll
  for (int i = 0; i < 16; i += 4) {
    const f32x4 d = *(const f32x4*)(xr + 16 * jq + i);
#pragma unroll
    for (int u = 0; u < 4; ++u) dl[i + u] = av[i + u] * (d[u] - delta_q);
  }
  // bottom-up inside the 16 leaves: depth 5 (8 nodes), 4 (4), 3 (2), 2 (1)
  float gv[15];
#pragma unroll
  for (int e = 3; e >= 0; --e)
#pragma unroll
    for (int i = 0; i < (1 << e); ++i) {
      const float al = dl[2 * i], ar = dl[2 * i + 1];
      gv[(1 << e) - 1 + i] = node_grad(xg[(1 << e) - 1 + i], al, ar);
      dl[i] = al + ar;
    }
  const float t16 = dl[0];                       // the depth-2 node's total
  const float t16o = __shfl_xor(t16, 1, 64);     // its sibling's
  const float p32 = t16 + t16o;                  // depth-1 node total
  const float p32o = __shfl_xor(p32, 2, 64);
  const float g1 = (jq & 1) ? node_grad(x1, t16o, t16) : node_grad(x1, t16, t16o);
  const float g0 = (jq >> 1) ? node_grad(x0, p32o, p32) : node_grad(x0, p32, p32o);
  E* gr = Gs + qi * PS;
#pragma unroll
  for (int e = 0; e < 4; ++e)
#pragma unroll
    for (int i = 0; i < (1 << e); ++i) gr[(1 << (2 + e)) - 1 + (jq << e) + i] = (E)gv[(1 << e) - 1 + i];
  if (!(jq & 1)) gr[1 + (jq >> 1)] = (E)g1;
  if (jq == 0) gr[0] = (E)g0;
  return p32 + p32o;
}

// dq_sub and chunk totals: one workgroup per 64 queries of one (batch, head).
template <typename E, int D>
__global__ __launch_bounds__(256, 2) void det_bwd_q_kernel(DetBwdArgs a) {
  using M = Mfma<E>;
  using TL = DbTiles<E, D>;
  constexpr int RS = TL::RS, XS = TL::XS, PS = TL::PS, NDT = D / 16;
  __shared__ __align__(16) E Ks[kDbCols * RS];
  __shared__ __align__(16) E Vs[kDbLeaves * RS];
  __shared__ __align__(16) float Xs[kDbQ * XS];
  __shared__ __align__(16) E Gs[kDbQ * PS];
  const int bh = blockIdx.y, bb = bh / a.H, h = bh - bb * a.H;
  const int l0 = blockIdx.x * kDbQ;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, col = lane & 15, g = lane >> 4;
  const int tt = a.T - 6, NC = 1 << tt;
  const int qi = tid >> 2, lq = l0 + qi;
  RowFrags<E, D> qa, ga;
  {
    const int l = l0 + 16 * w + col;
    const bool in = l < a.L;
    qa.load(in ? (const E*)a.q + bb * a.qsb + (int64_t)l * a.qsl + h * a.qsh : nullptr, g);
    ga.load(in ? (const E*)a.g + bb * a.gsb + (int64_t)l * a.gsl + h * a.gsh : nullptr, g);
  }
  const bool qin = lq < a.L;
  const float lse_q = a.causal && qin ? a.lse[(int64_t)bh * a.L + lq] : 0.f;
  const float delta_q = a.causal && qin ? a.delta[(int64_t)bh * a.L + lq] : 0.f;
  if (tid < kDbQ) Gs[tid * PS + kDbLeaves - 1] = (E)0.f;  // column 63 pads the 63 nodes to 64
  f32x4 dacc[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) dacc[i] = zero4();
  int nchunk = NC;
  if (a.causal) nchunk = min(NC, (min(l0 + kDbQ, a.L) - 1) / kDbLeaves + 1);
  for (int r = 0; r < nchunk; ++r) {
    __syncthreads();
    stage_chunk<E, D>(a, bb, h, r, tt, Ks, Vs, tid);
    __syncthreads();
    const float tot = tile_grad<E, D>(qa, ga, Ks, Vs, Xs, Gs, nullptr, r, tt, lq, lse_q, delta_q, a.causal, tid);
    if ((tid & 3) == 0 && qin) a.achunk[((int64_t)bh * a.L + lq) * NC + r] = tot;
    // dq += G K_sub over the chunk's 63 nodes (rows tt .. tt + 62 of Ks; row tt + 63 is padding or
    // another column whose G is zero)
#pragma unroll
    for (int ks = 0; ks < kDbLeaves / M::K; ++ks) {
      const typename M::frag ga_ = ld_frag(Gs + (16 * w + col) * PS + ks * M::K + M::KPL * g);
      const int ka = ks * M::K + M::KPL * g;
#pragma unroll
      for (int nd = 0; nd < NDT; ++nd) dacc[nd] = M::mma(ga_, tr_frag(Ks + tt * RS, RS, ka, ka + 4, 16 * nd, lane), dacc[nd]);
    }
  }
  if (a.causal) {  // chunks past the tile's last query: zero totals
    for (int r = nchunk; r < NC; ++r)
      if ((tid & 3) == 0 && qin) a.achunk[((int64_t)bh * a.L + lq) * NC + r] = 0.f;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int l = l0 + 16 * w + 4 * g + i;
    if (l >= a.L) continue;
    float* o = a.dq + ((int64_t)bh * a.L + l) * D + col;
#pragma unroll
    for (int nd = 0; nd < NDT; ++nd) o[16 * nd] = dacc[nd][i];
  }
}

// dv and the chunk's subtree rows of dk: one workgroup per (chunk, batch*head).
template <typename E, int D>
__global__ __launch_bounds__(256, D <= 64 ? 2 : 1) void det_bwd_kv_kernel(DetBwdArgs a) {
  using M = Mfma<E>;
  using TL = DbTiles<E, D>;
  constexpr int RS = TL::RS, XS = TL::XS, PS = TL::PS, NDT = D / 16, KS = D / M::K;
  __shared__ __align__(16) E Ks[kDbCols * RS];
  __shared__ __align__(16) E Vs[kDbLeaves * RS];
  __shared__ __align__(16) E Qs[kDbQ * RS];
  __shared__ __align__(16) E Gds[kDbQ * RS];
  __shared__ __align__(16) float Xs[kDbQ * XS];
  __shared__ __align__(16) E Gs[kDbQ * PS];
  __shared__ __align__(16) E Ws[kDbQ * PS];
  const int r = blockIdx.x, bh = blockIdx.y, bb = bh / a.H, h = bh - bb * a.H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, col = lane & 15, g = lane >> 4;
  const int tt = a.T - 6;
  if (tid < kDbQ) Gs[tid * PS + kDbLeaves - 1] = (E)0.f;
  stage_chunk<E, D>(a, bb, h, r, tt, Ks, Vs, tid);
  f32x4 vacc[NDT], kacc[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) {
    vacc[i] = zero4();
    kacc[i] = zero4();
  }
  const int ntile = (a.L + kDbQ - 1) / kDbQ;
  const int t0 = a.causal ? min(ntile, r * kDbLeaves / kDbQ) : 0;  // earlier tiles see none of the chunk
  for (int t = t0; t < ntile; ++t) {
    const int l0 = t * kDbQ, lq = l0 + (tid >> 2);
    const bool qin = lq < a.L;
    RowFrags<E, D> qa, ga;
    {
      const int l = l0 + 16 * w + col;
      const bool in = l < a.L;
      qa.load(in ? (const E*)a.q + bb * a.qsb + (int64_t)l * a.qsl + h * a.qsh : nullptr, g);
      ga.load(in ? (const E*)a.g + bb * a.gsb + (int64_t)l * a.gsl + h * a.gsh : nullptr, g);
    }
    const float lse_q = a.causal && qin ? a.lse[(int64_t)bh * a.L + lq] : 0.f;
    const float delta_q = a.causal && qin ? a.delta[(int64_t)bh * a.L + lq] : 0.f;
    __syncthreads();  // the previous tile's Qs / Gds / Gs / Ws are consumed
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      *(typename M::frag*)(Qs + (16 * w + col) * RS + ks * M::K + M::KPL * g) = qa.f[ks];
      *(typename M::frag*)(Gds + (16 * w + col) * RS + ks * M::K + M::KPL * g) = ga.f[ks];
    }
    tile_grad<E, D>(qa, ga, Ks, Vs, Xs, Gs, Ws, r, tt, lq, lse_q, delta_q, a.causal, tid);
    __syncthreads();
    // wave w: leaves / nodes 16w .. 16w + 15 against all 64 queries
#pragma unroll
    for (int ks = 0; ks < kDbQ / M::K; ++ks) {
      const int ka = ks * M::K + M::KPL * g;
      const typename M::frag wa = tr_frag(Ws, PS, ka, ka + 4, 16 * w, lane);
      const typename M::frag gaa = tr_frag(Gs, PS, ka, ka + 4, 16 * w, lane);
#pragma unroll
      for (int nd = 0; nd < NDT; ++nd) {
        vacc[nd] = M::mma(wa, tr_frag(Gds, RS, ka, ka + 4, 16 * nd, lane), vacc[nd]);
        kacc[nd] = M::mma(gaa, tr_frag(Qs, RS, ka, ka + 4, 16 * nd, lane), kacc[nd]);
      }
    }
  }
  E* dv = (E*)a.dv;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = 16 * w + 4 * g + i;  // leaf of the chunk, and subtree node
    const int64_t tok = (int64_t)r * kDbLeaves + m;
    E* o = dv + bb * a.dvsb + tok * a.dvsl + h * a.dvsh + col;
#pragma unroll
    for (int nd = 0; nd < NDT; ++nd) o[16 * nd] = (E)vacc[nd][i];
    if (m < kDbLeaves - 1) {
      const int node = chunk_node(tt + m, r, tt);
      float* dk = a.dkn + (((int64_t)node * a.B + bb) * a.H + h) * D + col;
#pragma unroll
      for (int nd = 0; nd < NDT; ++nd) dk[16 * nd] = kacc[nd][i];
    }
  }
}

template <typename E, int D>
static hipError_t det_bwd_t(const DetBwdArgs& a, hipStream_t st) {
  const int NC = 1 << (a.T - 6);
  hipLaunchKernelGGL((det_bwd_q_kernel<E, D>), dim3((unsigned)((a.L + kDbQ - 1) / kDbQ), (unsigned)(a.B * a.H)),
                     dim3(256), 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((det_bwd_kv_kernel<E, D>), dim3((unsigned)NC, (unsigned)(a.B * a.H)), dim3(256), 0, st, a);
  return hipGetLastError();
}

template <typename E>
static hipError_t det_bwd_d(const DetBwdArgs& a, int D, hipStream_t st) {
  switch (D) {
    case 32: return det_bwd_t<E, 32>(a, st);
    case 64: return det_bwd_t<E, 64>(a, st);
    case 96: return det_bwd_t<E, 96>(a, st);
    default: return det_bwd_t<E, 128>(a, st);
  }
}

hipError_t launch_det_stream_bwd(int dtype, const void* q, const int64_t* qs, const void* gout, const int64_t* gs,
                                 const void* kn, const int64_t* ks, const void* v, const int64_t* vs, const float* lse,
                                 const float* delta, float* dq, float* achunk, float* dkn, void* dv,
                                 const int64_t* dvs, int B, int L, int H, int D, int T, int causal, hipStream_t st) {
  DetBwdArgs a;
  a.q = q;
  a.qsb = qs[0]; a.qsl = qs[1]; a.qsh = qs[2];
  a.g = gout;
  a.gsb = gs[0]; a.gsl = gs[1]; a.gsh = gs[2];
  a.kn = kn;
  a.ksb = ks[0]; a.ksn = ks[1]; a.ksh = ks[2];
  a.v = v;
  a.vsb = vs[0]; a.vsl = vs[1]; a.vsh = vs[2];
  a.lse = lse;
  a.delta = delta;
  a.dq = dq;
  a.achunk = achunk;
  a.dkn = dkn;
  a.dv = dv;
  a.dvsb = dvs[0]; a.dvsl = dvs[1]; a.dvsh = dvs[2];
  a.B = B;
  a.L = L;
  a.H = H;
  a.T = T;
  a.causal = causal;
  if (B * H == 0) return hipSuccess;
  return dtype == TA_BF16 ? det_bwd_d<bf16>(a, D, st) : det_bwd_d<f16>(a, D, st);
}

}  // namespace ta
