// K4b: tree part of the backward (the reference's per-depth grad_logit and
// q/k accumulation, _autograd.py:789-856 and
// accumulate_qk_non_causal_all_depths_prepared.cu:104-161), deterministic:
//
//  * dlogp_s = w_s (delta_s - sum_s' w_s' delta_s'), delta from the leaf
//    backward (softmax-over-samples adjoint, _autograd.py:791-794);
//  * at depth d a sample at node i with chosen child j* contributes
//    dx_j = dlogp_s (1[j = j*] - p_j) to every child logit j of i (zero where
//    the logit was clamped); per query these are summed into G (queries x
//    child summaries of one column chunk) in LDS;
//  * tree_dq_kernel:   dq = sum_pairs dq_pair + sum_chunks G C_chunk     (MFMA)
//  * tree_dsum_kernel: dC_chunk = sum_queries G^T Q per query split      (MFMA)
//    and dsum_reduce_kernel adds the splits in order;
//  * pool_adjoint_kernel: dk = dk_leaf + (summaries map)^T dC, which for
//    compat summaries is the transpose of the reference's Haar keys
//    (_treeattn_common.py:70-86).
// The causal correction adds the same -log A_root to every sample of a
// query; since sum_s dlogp_s = 0 it has no gradient.
#include "launch.h"

namespace ta {

struct TreeArgs {
  Geo geo;
  int L, N, H, S, D, causal, mode;
  float maxhalf;
  const void* q;
  int64_t qsb, qsl, qsh;
  const float* weights;
  int64_t wsb, wsl, wsh;
  const void* sum_hi;  // E (BH, NS, D) (float inputs: the float summaries)
  const void* sum_t;   // E (BH, D, NS)
  const int* leaf;
  const int* slot_leaf;
  const int* slot_count;
  const float* delta;
  const void* dq_part;
  float* dlogp;
  void* dq;
  float* dsum_part;
  float* dsum;
  const float* dk_leaf;
  void* dk;
  int64_t ksb, ksl, ksh;
  int qsplit;
};

template <typename E>
__device__ __forceinline__ void cp8(E* o, const E* p) {
  if constexpr (sizeof(E) == 2) {
    *(uint4*)o = *(const uint4*)p;
  } else {
    *(float4*)o = *(const float4*)p;
    *(float4*)(o + 4) = *(const float4*)(p + 4);
  }
}
template <typename E>
__device__ __forceinline__ void z8(E* o) {
  if constexpr (sizeof(E) == 2) {
    *(uint4*)o = make_uint4(0, 0, 0, 0);
  } else {
    *(float4*)o = make_float4(0, 0, 0, 0);
    *(float4*)(o + 4) = make_float4(0, 0, 0, 0);
  }
}

__device__ __forceinline__ float clamp_h(float x, float m) { return fminf(fmaxf(x, -m), m); }

// Raw child logits of level `lam`, columns [c0, c0+ncols), into Xs[64][kChunk].
template <typename E, int D>
__device__ __forceinline__ void logits_tile(const E* Qs, float* Xs, const E* sum, int64_t row0, int ncols, int lane,
                                            int w) {
  using M = Mfma<E>;
  const int col = lane & 15, g = lane >> 4;
  const int ntiles = (ncols + 15) >> 4;
  for (int nt = 0; nt < ntiles; ++nt) {
    f32x4 c = zero4();
    const E* bp = sum + (row0 + nt * 16 + col) * D + M::KPL * g;
    const E* ap = Qs + (16 * w + col) * D + M::KPL * g;
#pragma unroll
    for (int ks = 0; ks < D / M::K; ++ks) c = M::mma(ld_frag(ap + ks * M::K), ld_frag(bp + ks * M::K), c);
#pragma unroll
    for (int r = 0; r < 4; ++r) Xs[(16 * w + 4 * g + r) * kChunk + nt * 16 + col] = c[r];
  }
}

// Adds query qi's dx terms for depth d and chunk [c0, c0+ncols) into
// G[qi*gq + col*gc].  Samples are visited in order (deterministic).
__device__ __forceinline__ void build_g_row(const Geo& G, int qi, int d, int c0, int ncols, int S, float maxhalf,
                                            const float* Xs, const int* lf, const float* dl, float* Gm, int gq,
                                            int gc) {
  const int b = G.b, T = G.T;
  for (int s = 0; s < S; ++s) {
    const int beta = lf[qi * S + s];
    const int i = beta / G.pw[T - d];
    const int base = b * i - c0;
    if (base < 0 || base >= ncols) continue;
    const int js = (beta / G.pw[T - 1 - d]) % b;
    const float* xr = Xs + qi * kChunk + base;
    float mx = -__builtin_inff();
    for (int j = 0; j < b; ++j) mx = fmaxf(mx, clamp_h(xr[j], maxhalf));
    float se = 0.f;
    for (int j = 0; j < b; ++j) se += expf(clamp_h(xr[j], maxhalf) - mx);
    const float lse = mx + logf(se);
    const float dls = dl[qi * S + s];
    for (int j = 0; j < b; ++j) {
      const float x = xr[j];
      const bool live = x >= -maxhalf && x <= maxhalf;
      const float p = expf(clamp_h(x, maxhalf) - lse);
      const float dx = live ? dls * ((j == js ? 1.f : 0.f) - p) : 0.f;
      Gm[qi * gq + (base + j) * gc] += dx;
    }
  }
}

template <typename E, int D>
__global__ __launch_bounds__(256) void tree_dq_kernel(TreeArgs a) {
  using M = Mfma<E>;
  extern __shared__ __align__(16) char smem[];
  const Geo& G = a.geo;
  const int bh = blockIdx.y, bb = bh / a.H, h = bh - bb * a.H;
  const int l0 = blockIdx.x * kQueryTile;
  const int nq = min(kQueryTile, a.L - l0);
  const int S = a.S, T = G.T;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, col = lane & 15, g = lane >> 4;
  const int64_t rows = G.NS;

  E* Qs = (E*)smem;                                  // [64][D]
  float* Xs = (float*)(Qs + kQueryTile * D);        // [64][kChunk] (also [64][D] staging)
  float* Gm = Xs + kQueryTile * kChunk;             // [64][kChunk]
  int* lf = (int*)(Gm + kQueryTile * kChunk);       // [64*S]
  float* dl = (float*)(lf + kQueryTile * S);        // [64*S]

  const E* q = (const E*)a.q;
  for (int e = tid; e < kQueryTile * D / 8; e += 256) {
    const int r = e / (D / 8), c = (e - r * (D / 8)) * 8;
    if (r < nq) cp8(Qs + r * D + c, q + bb * a.qsb + (int64_t)(l0 + r) * a.qsl + h * a.qsh + c);
    else z8(Qs + r * D + c);
  }
  // dlogp per sample, one wavefront per query
  for (int qi = w; qi < kQueryTile; qi += 4) {
    const bool act = lane < S && qi < nq;
    const int l = l0 + qi;
    const int64_t qh = ((int64_t)bb * a.L + l) * a.H + h;
    int beta = 0;
    float wt = 0.f, dlt = 0.f;
    if (act) {
      beta = a.leaf[qh * S + lane];
      wt = a.weights[bb * a.wsb + (int64_t)l * a.wsl + h * a.wsh + lane];
      const int n = a.slot_count[qh];
      int u = 0;
      for (int j = 0; j < n; ++j)
        if (a.slot_leaf[qh * S + j] == beta) u = j;
      dlt = a.delta[qh * S + u];
    }
    const float tot = wave_sum(wt * dlt);
    const float dls = wt * (dlt - tot);
    if (lane < S) {
      lf[qi * S + lane] = beta;
      dl[qi * S + lane] = act ? dls : 0.f;
      if (act) a.dlogp[qh * S + lane] = dls;
    }
  }
  __syncthreads();

  f32x4 dacc[D / 16];
#pragma unroll
  for (int nd = 0; nd < D / 16; ++nd) dacc[nd] = zero4();
  const E* sum_hi = (const E*)a.sum_hi;
  const E* sum_t = (const E*)a.sum_t;
  for (int d = 0; d < T; ++d) {
    const int lam = d + 1, lvl = G.pw[lam];
    for (int c0 = 0; c0 < lvl; c0 += kChunk) {
      const int ncols = min(kChunk, lvl - c0);
      logits_tile<E, D>(Qs, Xs, sum_hi, (int64_t)bh * rows + G.off[lam] + c0, ncols, lane, w);
      for (int e = tid; e < kQueryTile * kChunk; e += 256) Gm[e] = 0.f;
      __syncthreads();
      if (tid < nq) build_g_row(G, tid, d, c0, ncols, S, a.maxhalf, Xs, lf, dl, Gm, kChunk, 1);
      __syncthreads();
      const int ksteps = (ncols + M::K - 1) / M::K;
#pragma unroll
      for (int nd = 0; nd < D / 16; ++nd) {
        const E* bp = sum_t + ((int64_t)bh * D + 16 * nd + col) * rows + G.off[lam] + c0 + M::KPL * g;
        const float* ap = Gm + (16 * w + col) * kChunk + M::KPL * g;
        for (int ks = 0; ks < ksteps; ++ks)
          dacc[nd] = M::mma(cvt_frag<E>(ap + ks * M::K, 1), ld_frag(bp + ks * M::K), dacc[nd]);
      }
      __syncthreads();
    }
  }
  // stage tree dq, add the leaf parts, write
  float* stage = Xs;
#pragma unroll
  for (int nd = 0; nd < D / 16; ++nd)
#pragma unroll
    for (int r = 0; r < 4; ++r) stage[(16 * w + 4 * g + r) * D + 16 * nd + col] = dacc[nd][r];
  __syncthreads();
  const E* dqp = (const E*)a.dq_part;
  E* dq = (E*)a.dq;
  for (int e = tid; e < nq * (D / 4); e += 256) {
    const int qi = e / (D / 4), d0 = (e - qi * (D / 4)) * 4;
    const int l = l0 + qi;
    const int64_t qh = ((int64_t)bb * a.L + l) * a.H + h;
    float acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = stage[qi * D + d0 + i];
    const int n = a.slot_count[qh];
    for (int u = 0; u < n; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] += tof(dqp[(qh * S + u) * D + d0 + i]);
    E* o = dq + bb * a.qsb + (int64_t)l * a.qsl + h * a.qsh + d0;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (E)acc[i];
  }
}

// grid (ncol, BH, qsplit).  Column chunk -> (level, c0).
template <typename E, int D>
__global__ __launch_bounds__(256) void tree_dsum_kernel(TreeArgs a) {
  using M = Mfma<E>;
  constexpr int NT = (kChunk / 16) * (D / 16) / 4;
  extern __shared__ __align__(16) char smem[];
  const Geo& G = a.geo;
  const int bh = blockIdx.y, bb = bh / a.H, h = bh - bb * a.H;
  const int split = blockIdx.z;
  const int S = a.S, T = G.T;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, col = lane & 15, g = lane >> 4;
  const int64_t rows = G.NS;

  int lam = 1, c0 = 0, rem = blockIdx.x;
  for (; lam <= T; ++lam) {
    const int nc = (G.pw[lam] + kChunk - 1) / kChunk;
    if (rem < nc) { c0 = rem * kChunk; break; }
    rem -= nc;
  }
  const int d = lam - 1;
  const int ncols = min(kChunk, G.pw[lam] - c0);

  E* Qs = (E*)smem;                              // [64][D]
  float* Xs = (float*)(Qs + kQueryTile * D);    // [64][kChunk]
  float* Gt = Xs + kQueryTile * kChunk;         // [kChunk][64]
  int* lf = (int*)(Gt + kQueryTile * kChunk);   // [64*S]
  float* dl = (float*)(lf + kQueryTile * S);    // [64*S]

  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = zero4();

  const int ntiles = (a.L + kQueryTile - 1) / kQueryTile;
  const int per = (ntiles + a.qsplit - 1) / a.qsplit;
  const int tt0 = split * per, tt1 = min(ntiles, tt0 + per);
  const E* q = (const E*)a.q;
  const E* sum_hi = (const E*)a.sum_hi;
  for (int tt = tt0; tt < tt1; ++tt) {
    const int l0 = tt * kQueryTile;
    const int nq = min(kQueryTile, a.L - l0);
    __syncthreads();
    for (int e = tid; e < kQueryTile * D / 8; e += 256) {
      const int r = e / (D / 8), c = (e - r * (D / 8)) * 8;
      if (r < nq) cp8(Qs + r * D + c, q + bb * a.qsb + (int64_t)(l0 + r) * a.qsl + h * a.qsh + c);
      else z8(Qs + r * D + c);
    }
    for (int e = tid; e < kQueryTile * S; e += 256) {
      const int qi = e / S, s = e - qi * S;
      if (qi < nq) {
        const int64_t qh = ((int64_t)bb * a.L + l0 + qi) * a.H + h;
        lf[e] = a.leaf[qh * S + s];
        dl[e] = a.dlogp[qh * S + s];
      } else {
        lf[e] = 0;
        dl[e] = 0.f;
      }
    }
    for (int e = tid; e < kQueryTile * kChunk; e += 256) Gt[e] = 0.f;
    __syncthreads();
    logits_tile<E, D>(Qs, Xs, sum_hi, (int64_t)bh * rows + G.off[lam] + c0, ncols, lane, w);
    __syncthreads();
    if (tid < nq) build_g_row(G, tid, d, c0, ncols, S, a.maxhalf, Xs, lf, dl, Gt, 1, kQueryTile);
    __syncthreads();
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int tile = w + 4 * t;
      const int mc = tile / (D / 16), nd = tile - mc * (D / 16);
      if (16 * mc >= ncols) continue;
      const float* ap = Gt + (16 * mc + col) * kQueryTile + M::KPL * g;
      const E* bp = Qs + (M::KPL * g) * D + 16 * nd + col;
#pragma unroll
      for (int ks = 0; ks < kQueryTile / M::K; ++ks)
        acc[t] = M::mma(cvt_frag<E>(ap + ks * M::K, 1), ld_frag_strided(bp + ks * M::K * D, D), acc[t]);
    }
  }
  float* out = a.dsum_part + ((int64_t)split * gridDim.y + bh) * rows * D;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int tile = w + 4 * t;
    const int mc = tile / (D / 16), nd = tile - mc * (D / 16);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int c = 16 * mc + 4 * g + r;
      if (c < ncols) out[(int64_t)(G.off[lam] + c0 + c) * D + 16 * nd + col] = acc[t][r];
    }
  }
}

// dsum = sum over query splits (in split order); rows outside any level are 0.
__global__ __launch_bounds__(256) void dsum_reduce_kernel(const float* __restrict__ part, float* __restrict__ dsum,
                                                          int64_t n, int qsplit, Geo G, int D) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n) return;
  const int64_t r = (e / D) % G.NS;
  int lam = 1;
  while (lam < G.T && r >= G.off[lam + 1]) ++lam;
  float s = 0.f;
  if (r - G.off[lam] < G.pw[lam])
    for (int k = 0; k < qsplit; ++k) s += part[(int64_t)k * n + e];
  dsum[e] = s;
}

// dk[b, t, h, :] = dk_leaf + sum over the summaries that include token t.
template <typename E>
__global__ __launch_bounds__(256) void pool_adjoint_kernel(TreeArgs a) {
  const Geo& G = a.geo;
  const int D = a.D;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (int64_t)a.N * D) return;
  const int bh = blockIdx.y, bb = bh / a.H, h = bh - bb * a.H;
  const int t = (int)(e / D), d = (int)(e - (int64_t)t * D);
  const int beta = t / G.LB;
  const float* ds = a.dsum + (int64_t)bh * G.NS * D + d;
  float acc = 0.f;
  if (a.mode == TA_TREE_NATURAL) {
    for (int lam = 1; lam <= G.T; ++lam) {
      const int per = G.NL / G.pw[lam];
      acc += ds[(int64_t)(G.off[lam] + beta / per) * D] / (2.f * (float)per);
    }
  } else {
    // compat: dcoef_n = (dC_left - dC_right)/2 for heap node n; the in-order
    // coefficient p = n+1 at level l = ctz(p) spans blocks [p - 2^l, p + 2^l)
    for (int l = 0; (1 << (l + 1)) <= G.NL; ++l) {
      const int wl = 1 << l;
      const int p = ((beta >> (l + 1)) << (l + 1)) + wl;
      const int nn = p - 1;
      const int dep = 31 - __clz(nn + 1);
      const int ip = nn + 1 - (1 << dep);
      const int64_t rl = G.off[dep + 1] + 2 * ip;
      const float dcoef = 0.5f * (ds[rl * D] - ds[(rl + 1) * D]);
      const float term = dcoef / (2.f * (float)wl);
      acc += beta < p ? term : -term;
    }
  }
  acc /= (float)G.LB;
  const int64_t th = ((int64_t)bb * a.N + t) * a.H + h;
  acc += a.dk_leaf[th * D + d];
  ((E*)a.dk)[bb * a.ksb + (int64_t)t * a.ksl + h * a.ksh + d] = (E)acc;
}

// Node-keys mode: dk[node n] = (dC_left - dC_right) / 2.
template <typename E>
__global__ __launch_bounds__(256) void nodekeys_adjoint_kernel(TreeArgs a) {
  const Geo& G = a.geo;
  const int D = a.D;
  const int K = G.NL - 1;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (int64_t)K * D) return;
  const int bh = blockIdx.y, bb = bh / a.H, h = bh - bb * a.H;
  const int nn = (int)(e / D), d = (int)(e - (int64_t)nn * D);
  const int dep = 31 - __clz(nn + 1);
  const int ip = nn + 1 - (1 << dep);
  const int64_t rl = G.off[dep + 1] + 2 * ip;
  const float* ds = a.dsum + (int64_t)bh * G.NS * D + d;
  ((E*)a.dk)[bb * a.ksb + (int64_t)nn * a.ksl + h * a.ksh + d] = (E)(0.5f * (ds[rl * D] - ds[(rl + 1) * D]));
}

int tree_dq_smem(const Plan& P) {
  return kQueryTile * (int)P.D * P.esize + 2 * kQueryTile * kChunk * 4 + kQueryTile * (int)P.S * 8;
}

template <typename E, int D>
static hipError_t tree_impl(const Plan& P, const void* q, const float* weights, const char* rec, void* dq, void* dk,
                            char* ws, hipStream_t st) {
  TreeArgs a;
  a.geo = P.geo;
  a.L = (int)P.L;
  a.N = (int)P.N;
  a.H = (int)P.H;
  a.S = (int)P.S;
  a.D = D;
  a.causal = P.p.causal;
  a.mode = P.p.tree_mode;
  a.maxhalf = 0.5f * P.p.max_logit;
  a.q = q;
  a.qsb = P.p.q_strides[0]; a.qsl = P.p.q_strides[1]; a.qsh = P.p.q_strides[2];
  a.weights = weights;
  a.wsb = P.p.w_strides[0]; a.wsl = P.p.w_strides[1]; a.wsh = P.p.w_strides[2];
  a.sum_hi = sizeof(E) == 2 ? (const void*)(rec + P.rec.sum_hi) : (const void*)(rec + P.rec.summaries);
  a.sum_t = rec + P.rec.sum_t;
  a.leaf = (const int*)(rec + P.rec.leaf);
  a.slot_leaf = (const int*)(rec + P.rec.slot_leaf);
  a.slot_count = (const int*)(rec + P.rec.slot_count);
  a.delta = (const float*)(ws + P.bws.delta);
  a.dq_part = ws + P.bws.dq_part;
  a.dlogp = (float*)(ws + P.bws.dlogp);
  a.dq = dq;
  a.dsum_part = (float*)(ws + P.bws.dsum_part);
  a.dsum = (float*)(ws + P.bws.dsum);
  a.dk_leaf = (const float*)(ws + P.bws.dk_leaf);
  a.dk = dk;
  a.ksb = P.p.k_strides[0]; a.ksl = P.p.k_strides[1]; a.ksh = P.p.k_strides[2];
  a.qsplit = P.qsplit;

  const int smem = tree_dq_smem(P);
  hipError_t e = hipFuncSetAttribute((const void*)tree_dq_kernel<E, D>, hipFuncAttributeMaxDynamicSharedMemorySize, smem);
  if (e != hipSuccess) return e;
  e = hipFuncSetAttribute((const void*)tree_dsum_kernel<E, D>, hipFuncAttributeMaxDynamicSharedMemorySize, smem);
  if (e != hipSuccess) return e;
  const unsigned qtiles = (unsigned)((P.L + kQueryTile - 1) / kQueryTile);
  hipLaunchKernelGGL((tree_dq_kernel<E, D>), dim3(qtiles, P.BH), dim3(256), smem, st, a);
  if (P.geo.T > 0) {
    hipLaunchKernelGGL((tree_dsum_kernel<E, D>), dim3(P.ncol, P.BH, P.qsplit), dim3(256), smem, st, a);
    const int64_t n = P.BH * (int64_t)P.geo.NS * D;
    hipLaunchKernelGGL(dsum_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       (const float*)a.dsum_part, a.dsum, n, P.qsplit, P.geo, D);
  }
  if (P.p.tree_mode == TA_TREE_NODEKEYS) {
    const int64_t n = (int64_t)(P.geo.NL - 1) * D;
    if (n > 0)
      hipLaunchKernelGGL(nodekeys_adjoint_kernel<E>, dim3((unsigned)((n + 255) / 256), P.BH), dim3(256), 0, st, a);
  } else {
    const int64_t n = P.N * D;
    hipLaunchKernelGGL(pool_adjoint_kernel<E>, dim3((unsigned)((n + 255) / 256), P.BH), dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

template <typename E>
static hipError_t tree_d(const Plan& P, const void* q, const float* w, const char* rec, void* dq, void* dk, char* ws,
                         hipStream_t st) {
  switch (P.D) {
    case 32: return tree_impl<E, 32>(P, q, w, rec, dq, dk, ws, st);
    case 64: return tree_impl<E, 64>(P, q, w, rec, dq, dk, ws, st);
    case 96: return tree_impl<E, 96>(P, q, w, rec, dq, dk, ws, st);
    default: return tree_impl<E, 128>(P, q, w, rec, dq, dk, ws, st);
  }
}

hipError_t launch_tree_bwd(const Plan& P, const void* q, const float* weights, const char* rec, void* dq, void* dk,
                           char* ws, hipStream_t st) {
  switch (P.p.dtype) {
    case TA_F32: return tree_d<float>(P, q, weights, rec, dq, dk, ws, st);
    case TA_BF16: return tree_d<bf16>(P, q, weights, rec, dq, dk, ws, st);
    default: return tree_d<f16>(P, q, weights, rec, dq, dk, ws, st);
  }
}

}  // namespace ta
