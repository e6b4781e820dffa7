// K2, reference causal mode: the reference's causal stochastic sampler and
// its exact head, on the reference tree (binary, one token per leaf).
//
// Restates _sample_paths_causal (_tree_mha.py:125-268) and the hybrid split
// of hierarchical_attention (:379-394).  One workgroup owns one query
// position t and every (batch, head, sample) lane of it, because the
// reference couples them: the boundary correction applies at depth d only
// while ALL lanes of the query sit on the boundary path (:204-207), a
// workgroup-wide AND here.
//   * Boundary leaf c = t.  Pass 1 (per batch, head): the boundary-path node
//     logits x_d and the bottom-up log-masses
//       M_d = logsumexp(M_{d+1} + logsig(on),  m_off + logsig(off)),  M_T = 0,
//     with m_off = -inf when the boundary turns left at d and log(#leaves of
//     the left subtree) when it turns right (:166-196).
//   * Pass 2, top-down: each lane's node logit x = q . k_node (= 2 q . c_left);
//     while every lane is on the boundary path the two log-probabilities get
//     the masses: left m_l + logsig(x) - M_d, right m_r + logsig(-x) - M_d
//     (:216-249); afterwards they are plain.  Gumbel-max with the caller's
//     uniforms or the counter RNG; first maximum wins.
//   * When L > S, queries t < S are answered exactly instead (:379-385): all
//     leaves n <= t become the query's slots, weighted by the softmax of their
//     path log-probabilities, so the leaf and tree kernels treat them like
//     sampled rows.
// The first depth at which the lanes are no longer all on the boundary path
// is saved per query (the backward needs it).  Dots run on the vector ALU in
// float32 against the float summaries (q . c_left = q . k / 2).
#include "launch.h"

namespace ta {

struct RefSampleArgs {
  Geo geo;
  int B, L, H, S, D, hybrid;
  const void* q;
  int64_t qsb, qsl, qsh;
  const float* sum32;
  const float* U;
  uint64_t seed;
  float* weights;
  int64_t wsb, wsl, wsh;
  int* leaf;
  int* slot_leaf;
  float* slot_weight;
  int* slot_count;
  int* dstar;
};

// logit of heap node (depth d, index i within the level): 2 q . c_left
template <typename E>
__device__ __forceinline__ float node_logit(const RefSampleArgs& a, const E* qrow, int bh, int d, int i) {
  const float* c = a.sum32 + ((int64_t)bh * a.geo.NS + a.geo.off[d + 1] + 2 * i) * a.D;
  return 2.f * dot_row(qrow, c, a.D);
}

__device__ __forceinline__ float uniform_ref(const RefSampleArgs& a, int64_t idx) {
  if (a.U) return a.U[idx];
  const Philox4 ph = philox4x32_10((uint64_t)idx >> 2, a.seed);
  const int wi = (int)(idx & 3);
  return word_to_uniform(wi == 0 ? ph.w[0] : wi == 1 ? ph.w[1] : wi == 2 ? ph.w[2] : ph.w[3]);
}

// grid L, block 256.  LDS: node/lp/key per lane (3 * BH*S) and the masses (BH*(T+1)).
template <typename E>
__global__ __launch_bounds__(256) void ref_sample_kernel(RefSampleArgs a) {
  extern __shared__ __align__(16) char smem[];
  const int t = blockIdx.x, tid = threadIdx.x;
  const int T = a.geo.T, S = a.S, H = a.H;
  const int nbh = a.B * H, nit = nbh * S;
  int* nd = (int*)smem;             // [nit] current node (index within its level)
  float* lp = (float*)(nd + nit);   // [nit] accumulated log-prob
  int* fl = (int*)(lp + nit);       // [nit] distinct-leaf key
  float* M = (float*)(fl + nit);    // [nbh][T+1] boundary log-masses
  const E* q = (const E*)a.q;
  auto qrow = [&](int bh) {
    const int bb = bh / H, h = bh - bb * H;
    return q + bb * a.qsb + (int64_t)t * a.qsl + h * a.qsh;
  };

  if (a.hybrid && t < S) {
    // exact head: leaves n <= t, log P(n) = sum_d logsig(+-x) along n's path
    const int nl = t + 1;
    for (int e = tid; e < nbh * nl; e += 256) {
      const int bh = e / nl, n = e - bh * nl;
      const E* qr = qrow(bh);
      float acc = 0.f;
      for (int d = 0; d < T; ++d) {
        const float x = node_logit(a, qr, bh, d, n >> (T - d));
        acc += ((n >> (T - 1 - d)) & 1) ? logsig(-x) : logsig(x);
      }
      lp[bh * S + n] = acc;
    }
    __syncthreads();
    for (int it = tid; it < nit; it += 256) {
      const int bh = it / S, s = it - bh * S;
      const int bb = bh / H, h = bh - bb * H;
      const int64_t qh = ((int64_t)bb * a.L + t) * H + h;
      const float* pq = lp + bh * S;
      float m = -__builtin_inff();
      for (int j = 0; j < nl; ++j) m = fmaxf(m, pq[j]);
      float sum = 0.f;
      for (int j = 0; j < nl; ++j) sum += expf(pq[j] - m);
      const float w = s < nl ? expf(pq[s] - m) / sum : 0.f;
      a.weights[bb * a.wsb + (int64_t)t * a.wsl + h * a.wsh + s] = w;
      a.leaf[qh * S + s] = s < nl ? s : -1;
      if (s < nl) {
        a.slot_leaf[qh * S + s] = s;
        a.slot_weight[qh * S + s] = w;
      }
      if (s == 0) a.slot_count[qh] = nl;
    }
    if (tid == 0) a.dstar[t] = T;
    return;
  }

  const int c = t;  // boundary leaf
  // pass 1: boundary-path logits, then the log-masses bottom-up (one thread per (batch, head))
  for (int e = tid; e < nbh * T; e += 256) {
    const int bh = e / T, d = e - bh * T;
    M[bh * (T + 1) + d] = node_logit(a, qrow(bh), bh, d, c >> (T - d));
  }
  __syncthreads();
  for (int bh = tid; bh < nbh; bh += 256) {
    float* Mb = M + bh * (T + 1);
    float m = 0.f;
    for (int d = T - 1; d >= 0; --d) {
      const int dir = (c >> (T - 1 - d)) & 1;
      const float x = Mb[d];
      const float on = dir ? logsig(-x) : logsig(x), off = dir ? logsig(x) : logsig(-x);
      const float a0 = m + on;
      float md = a0;
      if (dir) {
        const float a1 = logf((float)(1 << (T - 1 - d))) + off;
        const float mx = fmaxf(a0, a1);
        md = mx + logf(expf(a0 - mx) + expf(a1 - mx));
      }
      Mb[d] = md;
      m = md;
    }
    Mb[T] = 0.f;
  }
  for (int it = tid; it < nit; it += 256) {
    nd[it] = 0;
    lp[it] = 0.f;
  }
  __syncthreads();

  // pass 2: top-down; corrected while every lane is on the boundary path
  int dst = T;
  for (int d = 0; d < T; ++d) {
    const int bnode = c >> (T - d);
    bool on = true;
    for (int it = tid; it < nit; it += 256) on = on && nd[it] == bnode;
    const bool corr = __syncthreads_and(on) != 0 && dst == T;
    if (!corr && dst == T) dst = d;
    const int dirb = (c >> (T - 1 - d)) & 1;
    const float lcount = logf((float)(1 << (T - 1 - d)));
    for (int it = tid; it < nit; it += 256) {
      const int bh = it / S, s = it - bh * S;
      const int bb = bh / H, h = bh - bb * H;
      const int node = nd[it];
      const float x = node_logit(a, qrow(bh), bh, d, node);
      float lpl = logsig(x), lpr = logsig(-x);
      if (corr) {
        const float mp = M[bh * (T + 1) + d], mc = M[bh * (T + 1) + d + 1];
        if (dirb == 0) {
          lpl = mc + lpl - mp;
          lpr = -__builtin_inff();
        } else {
          lpl = lcount + lpl - mp;
          lpr = mc + lpr - mp;
        }
      }
      const int64_t ub = (((((int64_t)bb * a.L + t) * H + h) * S + s) * T + d) * 2;
      const float gl = -logf(-logf(uniform_ref(a, ub)));
      const float gr = -logf(-logf(uniform_ref(a, ub + 1)));
      const bool right = lpr + gr > lpl + gl;
      lp[it] += right ? lpr : lpl;
      nd[it] = 2 * node + (right ? 1 : 0);
    }
    __syncthreads();
  }
  if (tid == 0) a.dstar[t] = dst;

  // weights (softmax over each (batch, head)'s samples) and distinct leaves
  for (int it = tid; it < nit; it += 256) {
    const int bh = it / S, s = it - bh * S;
    const int* lq = nd + bh * S;
    const int me = lq[s];
    bool first = true;
    for (int j = 0; j < s; ++j) first = first && lq[j] != me;
    fl[it] = first ? me : 0x7fffffff;
  }
  __syncthreads();
  for (int it = tid; it < nit; it += 256) {
    const int bh = it / S, s = it - bh * S;
    const int bb = bh / H, h = bh - bb * H;
    const int64_t qh = ((int64_t)bb * a.L + t) * H + h;
    const int* lq = nd + bh * S;
    const float* pq = lp + bh * S;
    const int* fq = fl + bh * S;
    const int me = lq[s];
    float m = -__builtin_inff();
    for (int j = 0; j < S; ++j) m = fmaxf(m, pq[j]);
    float sum = 0.f, tot = 0.f;
    for (int j = 0; j < S; ++j) {
      const float e = expf(pq[j] - m);
      sum += e;
      if (lq[j] == me) tot += e;
    }
    a.weights[bb * a.wsb + (int64_t)t * a.wsl + h * a.wsh + s] = expf(pq[s] - m) / sum;
    a.leaf[qh * S + s] = me;
    if (fq[s] != 0x7fffffff) {
      int rank = 0;
      for (int j = 0; j < S; ++j) rank += fq[j] < me;
      a.slot_leaf[qh * S + rank] = me;
      a.slot_weight[qh * S + rank] = tot / sum;
    }
    if (s == 0) {
      int cnt = 0;
      for (int j = 0; j < S; ++j) cnt += fq[j] != 0x7fffffff;
      a.slot_count[qh] = cnt;
    }
  }
}

int ref_sample_smem(const Plan& P) {
  return (int)(3 * P.BH * P.S * 4 + P.BH * (P.geo.T + 1) * 4);
}

template <typename E>
static hipError_t ref_sample_impl(const Plan& P, const void* q, const float* U, uint64_t seed, float* weights,
                                  char* rec, hipStream_t st) {
  RefSampleArgs a;
  a.geo = P.geo;
  a.B = (int)P.B;
  a.L = (int)P.L;
  a.H = (int)P.H;
  a.S = (int)P.S;
  a.D = (int)P.D;
  a.hybrid = P.L > P.S;
  a.q = q;
  a.qsb = P.p.q_strides[0];
  a.qsl = P.p.q_strides[1];
  a.qsh = P.p.q_strides[2];
  a.sum32 = (const float*)(rec + P.rec.summaries);
  a.U = U;
  a.seed = seed;
  a.weights = weights;
  a.wsb = P.p.w_strides[0];
  a.wsl = P.p.w_strides[1];
  a.wsh = P.p.w_strides[2];
  a.leaf = (int*)(rec + P.rec.leaf);
  a.slot_leaf = (int*)(rec + P.rec.slot_leaf);
  a.slot_weight = (float*)(rec + P.rec.slot_weight);
  a.slot_count = (int*)(rec + P.rec.slot_count);
  a.dstar = (int*)(rec + P.rec.dstar);
  const int smem = ref_sample_smem(P);
  hipError_t e = hipFuncSetAttribute((const void*)ref_sample_kernel<E>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     smem);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(ref_sample_kernel<E>, dim3((unsigned)P.L), dim3(256), smem, st, a);
  return hipGetLastError();
}

hipError_t launch_ref_sample(const Plan& P, const void* q, const float* U, uint64_t seed, float* weights, char* rec,
                             hipStream_t st) {
  switch (P.p.dtype) {
    case TA_F32: return ref_sample_impl<float>(P, q, U, seed, weights, rec, st);
    case TA_BF16: return ref_sample_impl<bf16>(P, q, U, seed, weights, rec, st);
    default: return ref_sample_impl<f16>(P, q, U, seed, weights, rec, st);
  }
}

}  // namespace ta
