// K2: per-query root-to-leaf path sampling.
//
// Generalizes _sample_paths_non_causal (_tree_mha.py:78-122) and the
// treeattn-cuda step kernel (sample_non_causal_paths.cu:54-128) to b-ary trees
// with leaf blocks.  One workgroup owns 64 consecutive queries of one
// (batch, head).  Per depth, the child logits of every node of that level are
// an MFMA tile Q (64 x D) x summaries^T staged in LDS (summaries split into
// hi + lo parts of the input type so the logits are float-accurate); then each
// (query, sample) takes its decision from LDS:
//   logp_j = log_softmax(clamp(x_j, +-max_logit/2)),  plus the causal
//   correction on the boundary path, direction = argmax_j(logp_j + g_j)
//   (first maximum wins), g = -log(-log u) from the caller's uniforms or the
// counter RNG.  Finally one wavefront per query (lane = sample) writes the
// softmax weights over samples (_tree_mha.py:396-399) and the ascending list
// of distinct sampled leaf blocks with their summed weights.
#include "launch.h"

namespace ta {

struct SampleArgs {
  Geo geo;
  int L, H, S, causal, coff;  // coff = N - L: causal offset of query positions
  float maxhalf;
  const void* q;
  int64_t qsb, qsl, qsh;
  const float* sum32;
  const void* sum_hi;
  const void* sum_lo;
  const float* U;
  uint64_t seed;
  float* weights;
  int64_t wsb, wsl, wsh;
  int* leaf;
  int* slot_leaf;
  float* slot_weight;
  int* slot_count;
};

constexpr int kDoneBit = 1 << 30;
constexpr int kXS = kChunk + 4;  // padded row stride (floats) of the logit tile

__device__ __forceinline__ float clampf(float x, float m) { return fminf(fmaxf(x, -m), m); }

template <typename E, int D>
__global__ __launch_bounds__(256) void sample_kernel(SampleArgs a) {
  extern __shared__ __align__(16) char smem[];
  const Geo& G = a.geo;
  const int bh = blockIdx.y, bb = bh / a.H, h = bh - bb * a.H;
  const int l0 = blockIdx.x * kQueryTile;
  const int nq = min(kQueryTile, a.L - l0);
  const int S = a.S, T = G.T, b = G.b, lb = G.lb;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t rows = G.NS;
  constexpr bool kLo = sizeof(E) == 2;

  float* Xs = (float*)smem;
  int* node = (int*)(Xs + kQueryTile * kXS);
  float* acc = (float*)(node + kQueryTile * S);
  float* logA = acc + kQueryTile * S;        // [64][T+1]
  float* xb = logA + kQueryTile * (T + 1);   // [64][T*b]

  // this wave's 16 query rows stay in registers as MFMA A fragments
  RowFrags<E, D> qf;
  {
    const int r = 16 * w + (lane & 15);
    qf.load(r < nq ? (const E*)a.q + bb * a.qsb + (int64_t)(l0 + r) * a.qsl + h * a.qsh : nullptr, lane >> 4);
  }
  for (int e = tid; e < kQueryTile * S; e += 256) {
    node[e] = 0;
    acc[e] = 0.f;
  }
  __syncthreads();

  const E* hi = (const E*)(sizeof(E) == 2 ? a.sum_hi : (const void*)a.sum32);
  const E* lo = (const E*)a.sum_lo;

  // Causal: allowed log-mass of each boundary-path node, bottom-up:
  // A_T = 1, A_d = sum_{j<j*} p_j + p_{j*} A_{d+1}.  The boundary nodes of
  // consecutive queries form one contiguous node range per depth, so their
  // child logits come from the same MFMA tile as the walk's.
  if (a.causal && T > 0) {
    const int nb = T * b;
    const int blk_lo = (l0 + a.coff) / G.LB, blk_hi = (l0 + nq - 1 + a.coff) / G.LB;
    for (int d = 0; d < T; ++d) {
      const int sh = lb * (T - d);
      const int c0 = (blk_lo >> sh) << lb;
      const int ncols = (((blk_hi >> sh) + 1) << lb) - c0;
      for (int cc = 0; cc < ncols; cc += kChunk) {
        const int nc = min(kChunk, ncols - cc);
        const int64_t r0 = (int64_t)bh * rows + G.off[d + 1] + c0 + cc;
        mfma_rows<E, D, kLo>(qf, Xs, kXS, hi, lo, r0, nc, r0, lane, w);
        __syncthreads();
        for (int qi = tid; qi < nq; qi += 256) {
          const int blk = (l0 + qi + a.coff) / G.LB;
          const int col = ((blk >> sh) << lb) - c0 - cc;
          if (col >= 0 && col < nc)
            for (int j = 0; j < b; ++j) xb[qi * nb + d * b + j] = clampf(Xs[qi * kXS + col + j], a.maxhalf);
        }
        __syncthreads();
      }
    }
    if (tid < nq) {
      const int blk = (l0 + tid + a.coff) / G.LB;
      float* la = logA + tid * (T + 1);
      la[T] = 0.f;
      for (int d = T - 1; d >= 0; --d) {
        const int js = (blk >> (lb * (T - 1 - d))) & (b - 1);
        const float* xs = xb + tid * nb + d * b;
        float mx = -__builtin_inff();
        for (int j = 0; j < b; ++j) mx = fmaxf(mx, xs[j]);
        float se = 0.f;
        for (int j = 0; j < b; ++j) se += expf(xs[j] - mx);
        const float lse = mx + logf(se);
        // terms: logp_j (j < js), logp_js + logA_{d+1}
        float tm = -__builtin_inff();
        for (int j = 0; j <= js; ++j) tm = fmaxf(tm, xs[j] - lse + (j == js ? la[d + 1] : 0.f));
        float ts = 0.f;
        for (int j = 0; j <= js; ++j) ts += expf(xs[j] - lse + (j == js ? la[d + 1] : 0.f) - tm);
        la[d] = tm + logf(ts);
      }
    }
    __syncthreads();
  }

  for (int d = 0; d < T; ++d) {
    const int lam = d + 1, lvl = G.pw[lam];
    for (int c0 = 0; c0 < lvl; c0 += kChunk) {
      const int ncols = min(kChunk, lvl - c0);
      const int64_t r0 = (int64_t)bh * rows + G.off[lam] + c0;
      mfma_rows<E, D, kLo>(qf, Xs, kXS, hi, lo, r0, ncols, r0, lane, w);
      __syncthreads();
      for (int it = tid; it < kQueryTile * S; it += 256) {
        const int qi = it / S;
        if (qi >= nq) continue;
        const int i = node[it];
        if (i & kDoneBit) continue;
        const int base = (i << lb) - c0;
        if (base < 0 || base >= ncols) continue;
        const int s = it - qi * S;
        const float* xr = Xs + qi * kXS + base;
        float mx = -__builtin_inff();
        for (int j = 0; j < b; ++j) mx = fmaxf(mx, clampf(xr[j], a.maxhalf));
        float se = 0.f;
        for (int j = 0; j < b; ++j) se += expf(clampf(xr[j], a.maxhalf) - mx);
        const float lse = mx + logf(se);
        bool onb = false;
        int js = 0;
        float la_d = 0.f, la_c = 0.f;
        if (a.causal) {
          const int blk = (l0 + qi + a.coff) / G.LB;
          if ((blk >> (lb * (T - d))) == i) {
            onb = true;
            js = (blk >> (lb * (T - 1 - d))) & (b - 1);
            la_d = logA[qi * (T + 1) + d];
            la_c = logA[qi * (T + 1) + d + 1];
          }
        }
        const int64_t ubase = (((((int64_t)bb * a.L + l0 + qi) * a.H + h) * S + s) * T + d) * b;
        uint64_t cached = ~0ull;
        Philox4 ph;
        float best = -__builtin_inff(), bl = 0.f;
        int bj = 0;
        for (int j = 0; j < b; ++j) {
          float lp = clampf(xr[j], a.maxhalf) - lse;
          if (onb) {
            if (j < js) lp -= la_d;
            else if (j == js) lp += la_c - la_d;
            else lp = -__builtin_inff();
          }
          float u;
          if (a.U) {
            u = a.U[ubase + j];
          } else {
            const int64_t idx = ubase + j;
            const uint64_t ctr = (uint64_t)idx >> 2;
            if (ctr != cached) {
              ph = philox4x32_10(ctr, a.seed);
              cached = ctr;
            }
            const int wi = (int)(idx & 3);
            u = word_to_uniform(wi == 0 ? ph.w[0] : wi == 1 ? ph.w[1] : wi == 2 ? ph.w[2] : ph.w[3]);
          }
          const float sc = lp - logf(-logf(u));
          if (sc > best) {
            best = sc;
            bj = j;
            bl = lp;
          }
        }
        node[it] = ((i << lb) + bj) | kDoneBit;
        acc[it] += bl;
      }
      __syncthreads();
    }
    for (int it = tid; it < kQueryTile * S; it += 256) node[it] &= ~kDoneBit;
    __syncthreads();
  }

  // weights and distinct leaf blocks, one wavefront per query
  for (int qi = w; qi < nq; qi += 4) {
    const int l = l0 + qi;
    const int64_t qh = ((int64_t)bb * a.L + l) * a.H + h;
    const bool act = lane < S;
    const int beta = act ? node[qi * S + lane] : 0x7fffffff;
    const float lp = act ? acc[qi * S + lane] : -__builtin_inff();
    const float m = wave_max(lp);
    const float ex = act ? expf(lp - m) : 0.f;
    const float wgt = ex / wave_sum(ex);
    if (act) {
      a.weights[bb * a.wsb + (int64_t)l * a.wsl + h * a.wsh + lane] = wgt;
      a.leaf[qh * S + lane] = beta;
    }
    bool first = act;
    for (int j = 0; j < S; ++j) {
      const int bj = __shfl(beta, j, 64);
      if (j < lane && bj == beta) first = false;
    }
    int rank = 0, cnt = 0;
    float tot = 0.f;
    for (int j = 0; j < S; ++j) {
      const int bj = __shfl(beta, j, 64);
      const int fj = __shfl((int)first, j, 64);
      const float wj = __shfl(wgt, j, 64);
      if (fj && bj < beta) ++rank;
      cnt += fj;
      if (bj == beta && j >= lane) tot += wj;
    }
    if (first) {
      a.slot_leaf[qh * S + rank] = beta;
      a.slot_weight[qh * S + rank] = tot;
    }
    if (lane == 0) a.slot_count[qh] = cnt;
  }
}

int sample_smem(const Plan& P) {
  const int T = P.geo.T, b = P.geo.b;
  return kQueryTile * kXS * 4 + kQueryTile * (int)P.S * 8 +
         kQueryTile * (T + 1) * 4 + kQueryTile * T * b * 4;
}

template <typename E, int D>
static hipError_t sample_impl(const Plan& P, const void* q, const float* U, uint64_t seed, float* weights,
                              char* rec, hipStream_t st) {
  SampleArgs a;
  a.geo = P.geo;
  a.L = (int)P.L;
  a.H = (int)P.H;
  a.S = (int)P.S;
  a.causal = P.p.causal;
  a.coff = (int)(P.N - P.L);
  a.maxhalf = 0.5f * P.p.max_logit;
  a.q = q;
  a.qsb = P.p.q_strides[0];
  a.qsl = P.p.q_strides[1];
  a.qsh = P.p.q_strides[2];
  a.sum32 = (const float*)(rec + P.rec.summaries);
  a.sum_hi = rec + P.rec.sum_hi;
  a.sum_lo = rec + P.rec.sum_lo;
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
  const int smem = sample_smem(P);
  hipError_t e = hipFuncSetAttribute((const void*)sample_kernel<E, D>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, smem);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((sample_kernel<E, D>), dim3((unsigned)((P.L + kQueryTile - 1) / kQueryTile), P.BH),
                     dim3(256), smem, st, a);
  return hipGetLastError();
}

template <typename E>
static hipError_t sample_d(const Plan& P, const void* q, const float* U, uint64_t seed, float* w, char* rec,
                           hipStream_t st) {
  switch (P.D) {
    case 32: return sample_impl<E, 32>(P, q, U, seed, w, rec, st);
    case 64: return sample_impl<E, 64>(P, q, U, seed, w, rec, st);
    case 96: return sample_impl<E, 96>(P, q, U, seed, w, rec, st);
    default: return sample_impl<E, 128>(P, q, U, seed, w, rec, st);
  }
}

hipError_t launch_sample(const Plan& P, const void* q, const float* U, uint64_t seed, float* weights,
                         char* rec, hipStream_t st) {
  switch (P.p.dtype) {
    case TA_F32: return sample_d<float>(P, q, U, seed, weights, rec, st);
    case TA_BF16: return sample_d<bf16>(P, q, U, seed, weights, rec, st);
    default: return sample_d<f16>(P, q, U, seed, weights, rec, st);
  }
}

}  // namespace ta
