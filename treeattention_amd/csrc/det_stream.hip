// Streaming forward of the deterministic (exact) mode on the reference tree
// (_tree_mha.py:271-321) for 16-bit inputs: the (L, N) weights are never
// materialized, memory is O(L D).
//
// One workgroup (four waves) owns 64 queries of one (batch, head); wave w owns
// queries 16w..16w+15.  The N = 2^T leaves are walked in chunks of 64 (a
// subtree rooted at depth tt = T - 6).  Per chunk r:
//   1. the chunk's node keys -- its tt ancestors, then its 63 internal nodes in
//      breadth-first order, padded to 80 columns -- and its 64 value rows are
//      staged in LDS;
//   2. X = Q K_cols^T by MFMA (each wave its 16 queries x 80 columns);
//   3. each thread (query t/4, leaves 16(t%4)..+15 of the chunk) forms the
//      leaf log-weights: the ancestors' log-sigmoids, the two shared subtree
//      decisions, then a four-level register expansion
//      (lp[2i + c] = lp[i] + logsig(+-x), logsig(-x) = logsig(x) - x);
//   4. non-causal: P = exp(lp) (the exact path probabilities, summing to one
//      over all leaves); causal: an online softmax over the leaves n <= l
//      (running max and sum per query, the accumulated output rescaled);
//   5. O += P V by MFMA, P in the input type (the reference casts the weights
//      to v's type before W V, _tree_mha.py:318).
// Causal tiles stop at the last chunk holding a leaf <= the tile's last query.
// The causal log-normalizer lse = max + log(sum) per query goes to `lse` for
// the backward.
#include "launch.h"

namespace ta {

constexpr int kDsQ = 64;      // queries per workgroup
constexpr int kDsLeaves = 64; // leaves per chunk
constexpr int kDsCols = 80;   // node columns per chunk: <= 9 ancestors + 63 subtree nodes, padded

// log sigmoid(x) = min(x, 0) - log(1 + exp(-|x|)) on the hardware exp2 / log2.
__device__ __forceinline__ float logsig_fast(float x) {
  const float e = __builtin_amdgcn_exp2f(-fabsf(x) * 1.4426950408889634f);
  return fminf(x, 0.f) - 0.69314718055994531f * __builtin_amdgcn_logf(1.f + e);
}
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

struct DetStreamArgs {
  const void* q;
  int64_t qsb, qsl, qsh;
  const void* kn;  // heap-ordered node keys, (batch, node, head) strides
  int64_t ksb, ksn, ksh;
  const void* v;
  int64_t vsb, vsl, vsh;
  void* out;
  int64_t osb, osl, osh;
  float* lse;  // (B, H, L) causal log-normalizer, or null
  int B, L, H, T, causal;
};

// Eight-element row padding: at D <= 64 three workgroups fit per CU.
template <typename E, int D>
__global__ __launch_bounds__(256, D <= 64 ? 3 : 2) void det_stream_fwd_kernel(DetStreamArgs a) {
  using M = Mfma<E>;
  constexpr int KS = D / M::K;
  constexpr int RS = D + 8;              // LDS row stride (elements) of the K and V tiles
  constexpr int XS = kDsCols + 4;        // float row stride of the logit tile
  constexpr int PS = kDsLeaves + 8;      // row stride (elements) of the weight tile
  constexpr int NDT = D / 16;
  __shared__ __align__(16) E Ks[kDsCols * RS];
  __shared__ __align__(16) E Vs[kDsLeaves * RS];
  __shared__ __align__(16) float Xs[kDsQ * XS];
  __shared__ __align__(16) E Ps[kDsQ * PS];
  __shared__ float alpha_s[kDsQ], sum_s[kDsQ];

  const int bh = blockIdx.y, bb = bh / a.H, h = bh - bb * a.H;
  const int l0 = blockIdx.x * kDsQ;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, col = lane & 15, g = lane >> 4;
  const int T = a.T, tt = T - 6, NC = 1 << tt, ncol = tt + kDsLeaves - 1;
  const int nct = (ncol + 15) >> 4;
  const E* q = (const E*)a.q;
  const E* kn = (const E*)a.kn;
  const E* v = (const E*)a.v;

  RowFrags<E, D> qa;  // this wave's 16 query rows (A operand)
  {
    const int l = l0 + 16 * w + col;
    qa.load(l < a.L ? q + bb * a.qsb + (int64_t)l * a.qsl + h * a.qsh : nullptr, g);
  }
  const int qi = tid >> 2, jq = tid & 3;  // weights: query qi of the tile, leaves 16 jq .. 16 jq + 15
  const int lq = l0 + qi;
  float m_run = -__builtin_inff(), s_run = 0.f;
  f32x4 oacc[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) oacc[i] = zero4();

  int nchunk = NC;
  if (a.causal) nchunk = min(NC, (min(l0 + kDsQ, a.L) - 1) / kDsLeaves + 1);
  // Chunk tiles travel global -> registers one chunk ahead -> LDS, so the
  // loads of chunk r + 1 are in flight while chunk r computes.
  constexpr int NKL = (kDsCols * (D / 8) + 255) / 256, NVL = (kDsLeaves * (D / 8) + 255) / 256;
  uint4 kreg[NKL], vreg[NVL];
  auto fetch = [&](int r) {
#pragma unroll
    for (int j = 0; j < NKL; ++j) {
      const int e = tid + 256 * j;
      const int cix = e / (D / 8), d0 = (e - cix * (D / 8)) * 8;
      int node = -1;
      if (cix < tt) {
        node = (1 << cix) - 1 + (r >> (tt - cix));
      } else if (cix < ncol) {
        const int m = cix - tt, dep = 31 - __builtin_clz(m + 1);
        node = (1 << (tt + dep)) - 1 + (r << dep) + (m + 1 - (1 << dep));
      }
      kreg[j] = (e < kDsCols * (D / 8) && node >= 0)
                    ? *(const uint4*)(kn + bb * a.ksb + (int64_t)node * a.ksn + h * a.ksh + d0)
                    : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < NVL; ++j) {
      const int e = tid + 256 * j;
      const int lf = e / (D / 8), d0 = (e - lf * (D / 8)) * 8;
      const int64_t tok = (int64_t)r * kDsLeaves + lf;
      vreg[j] = e < kDsLeaves * (D / 8) ? *(const uint4*)(v + bb * a.vsb + tok * a.vsl + h * a.vsh + d0)
                                         : make_uint4(0, 0, 0, 0);
    }
  };
  fetch(0);
  for (int r = 0; r < nchunk; ++r) {
    __syncthreads();  // the previous chunk's tiles are consumed
#pragma unroll
    for (int j = 0; j < NKL; ++j) {
      const int e = tid + 256 * j;
      if (e < kDsCols * (D / 8)) *(uint4*)(Ks + (e / (D / 8)) * RS + (e % (D / 8)) * 8) = kreg[j];
    }
#pragma unroll
    for (int j = 0; j < NVL; ++j) {
      const int e = tid + 256 * j;
      if (e < kDsLeaves * (D / 8)) *(uint4*)(Vs + (e / (D / 8)) * RS + (e % (D / 8)) * 8) = vreg[j];
    }
    __syncthreads();
    if (r + 1 < nchunk) fetch(r + 1);

    // node logits of this wave's 16 queries: X^T tiles (node rows x query
    // columns), so each lane holds four consecutive columns of one query's
    // row -- one 16-byte store.  The logit and weight tiles' rows of these
    // queries are written and read by this wave only (in program order), so
    // only the chunk staging needs workgroup barriers.
    for (int ct = 0; ct < nct; ++ct) {
      f32x4 x = zero4();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) x = M::mma(ld_frag(Ks + (16 * ct + col) * RS + ks * M::K + M::KPL * g), qa.f[ks], x);
      *(f32x4*)(Xs + (16 * w + col) * XS + 16 * ct + 4 * g) = x;
    }

    // leaf log-weights of query qi, leaves 16 jq .. 16 jq + 15
    const float* xr = Xs + qi * XS;
    float av[16];
    {
      float pre = 0.f;
      for (int d = 0; d < tt; ++d) {
        const float x = xr[d], ls = logsig_fast(x);
        pre += ((r >> (tt - 1 - d)) & 1) ? ls - x : ls;
      }
      const float x0 = xr[tt], x1 = xr[tt + 1 + (jq >> 1)];
      const float l0s = logsig_fast(x0), l1s = logsig_fast(x1);
      pre += (jq >> 1) ? l0s - x0 : l0s;
      pre += (jq & 1) ? l1s - x1 : l1s;
      av[0] = pre;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int n0 = tt + (1 << (2 + e)) - 1 + (jq << e);  // column of the first node of this level
#pragma unroll
        for (int i = (1 << e) - 1; i >= 0; --i) {  // descending: a[2i], a[2i+1] overwrite nothing unread
          const float x = xr[n0 + i], ls = logsig_fast(x);
          av[2 * i + 1] = av[i] + ls - x;
          av[2 * i] = av[i] + ls;
        }
      }
    }
    float pv[16];
    const int nb = r * kDsLeaves + 16 * jq;  // global leaf index of av[0]
    if (a.causal) {
      float cm = -__builtin_inff();
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (nb + i <= lq) cm = fmaxf(cm, av[i]);
      cm = fmaxf(cm, __shfl_xor(cm, 1, 64));
      cm = fmaxf(cm, __shfl_xor(cm, 2, 64));
      const float mn = fmaxf(m_run, cm);
      const float al = (mn == -__builtin_inff() || m_run == -__builtin_inff()) ? (mn == m_run ? 1.f : 0.f)
                                                                                : exp_fast(m_run - mn);
      float ps = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        pv[i] = (nb + i <= lq) ? exp_fast(av[i] - mn) : 0.f;
        ps += pv[i];
      }
      ps += __shfl_xor(ps, 1, 64);
      ps += __shfl_xor(ps, 2, 64);
      s_run = s_run * al + ps;
      m_run = mn;
      if (jq == 0) alpha_s[qi] = al;
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) pv[i] = exp_fast(av[i]);
    }
    {
      typedef __attribute__((ext_vector_type(8))) E e8;
      e8 p0, p1;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        p0[i] = (E)pv[i];
        p1[i] = (E)pv[8 + i];
      }
      *(e8*)(Ps + qi * PS + 16 * jq) = p0;
      *(e8*)(Ps + qi * PS + 16 * jq + 8) = p1;
    }

    // O (this wave's 16 queries x D) = alpha O + P V
    if (a.causal) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float f = alpha_s[16 * w + 4 * g + i];
#pragma unroll
        for (int nd = 0; nd < NDT; ++nd) oacc[nd][i] *= f;
      }
    }
#pragma unroll
    for (int ks = 0; ks < kDsLeaves / M::K; ++ks) {
      const typename M::frag pa = ld_frag(Ps + (16 * w + col) * PS + ks * M::K + M::KPL * g);
      const int ka = ks * M::K + M::KPL * g;
#pragma unroll
      for (int nd = 0; nd < NDT; ++nd) oacc[nd] = M::mma(pa, tr_frag(Vs, RS, ka, ka + 4, 16 * nd, lane), oacc[nd]);
    }
  }

  if (a.causal && jq == 0) {
    sum_s[qi] = s_run;
    if (a.lse && lq < a.L) a.lse[(int64_t)bh * a.L + lq] = m_run + __logf(s_run);
  }
  __syncthreads();
  E* out = (E*)a.out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int qr = 16 * w + 4 * g + i, l = l0 + qr;
    if (l >= a.L) continue;
    const float inv = a.causal ? 1.f / sum_s[qr] : 1.f;
    E* o = out + bb * a.osb + (int64_t)l * a.osl + h * a.osh + col;
#pragma unroll
    for (int nd = 0; nd < NDT; ++nd) o[16 * nd] = (E)(oacc[nd][i] * inv);
  }
}

template <typename E, int D>
static hipError_t det_stream_t(const DetStreamArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)((a.L + kDsQ - 1) / kDsQ), (unsigned)(a.B * a.H));
  hipLaunchKernelGGL((det_stream_fwd_kernel<E, D>), grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

template <typename E>
static hipError_t det_stream_d(const DetStreamArgs& a, int D, hipStream_t st) {
  switch (D) {
    case 32: return det_stream_t<E, 32>(a, st);
    case 64: return det_stream_t<E, 64>(a, st);
    case 96: return det_stream_t<E, 96>(a, st);
    default: return det_stream_t<E, 128>(a, st);
  }
}

hipError_t launch_det_stream_fwd(int dtype, const void* q, const int64_t* qs, const void* kn, const int64_t* ks,
                                 const void* v, const int64_t* vs, void* out, const int64_t* os, float* lse, int B,
                                 int L, int H, int D, int T, int causal, hipStream_t st) {
  DetStreamArgs a;
  a.q = q;
  a.qsb = qs[0]; a.qsl = qs[1]; a.qsh = qs[2];
  a.kn = kn;
  a.ksb = ks[0]; a.ksn = ks[1]; a.ksh = ks[2];
  a.v = v;
  a.vsb = vs[0]; a.vsl = vs[1]; a.vsh = vs[2];
  a.out = out;
  a.osb = os[0]; a.osl = os[1]; a.osh = os[2];
  a.lse = lse;
  a.B = B;
  a.L = L;
  a.H = H;
  a.T = T;
  a.causal = causal;
  if (L == 0 || B * H == 0) return hipSuccess;
  return dtype == TA_BF16 ? det_stream_d<bf16>(a, D, st) : det_stream_d<f16>(a, D, st);
}

}  // namespace ta
