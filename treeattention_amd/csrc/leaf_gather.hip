// Leaf stage for trees with one token per leaf (leaf_block 1, the reference's
// own tree): a sampled leaf's output is its value row, so the forward is the
// reference's weighted value gather (_tree_mha.py:401-407,
// weighted_value_sum.cu:8-47) and the backward needs only
//   delta_u = dout_l . v[leaf_u]          (per distinct leaf of a query)
//   dv[n]   = sum_{(l, u) -> n} W_u dout_l   (the leaf's bucket, in order)
// (scatter_weighted_grad_v.cu:9-54 without atomics), both in one pass over
// the leaf buckets; the leaf softmax over one key has no gradient, so there
// is no leaf dq or dk.
#include "launch.h"

namespace ta {

template <typename E>
__device__ __forceinline__ void load8f(float* o, const E* p) {
  if constexpr (sizeof(E) == 2) {
    typedef __attribute__((ext_vector_type(8))) E e8;
    const e8 v = *(const e8*)p;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (float)v[i];
  } else {
    const float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  }
}
template <typename E>
__device__ __forceinline__ void store8f(E* o, const float* v) {
  if constexpr (sizeof(E) == 2) {
    typedef __attribute__((ext_vector_type(8))) E e8;
    e8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (E)v[i];
    *(e8*)o = r;
  } else {
    *(float4*)o = make_float4(v[0], v[1], v[2], v[3]);
    *(float4*)(o + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
}

struct GatherArgs {
  int L, N, H, S, D;
  const void* v;
  int64_t vsb, vsl, vsh;
  const void* g;  // output gradient
  int64_t gsb, gsl, gsh;
  void* out;      // forward output / dv
  int64_t osb, osl, osh;
  const int* slot_leaf;
  const float* slot_weight;
  const int* slot_count;
  const int* order;
  const int* block_start;
  float* delta;
  float* acc32;   // chunked problem: float (B, L|N, H, D) rows, written (first) or added to
  int first;
};

// out[b, l, h, :] = sum over the query's distinct leaves (slot order) of
// W_u v[leaf_u]; one thread per (query, 8 head dims) of (batch, head)s
// bh0 .. bh0 + nrows / L - 1.
template <typename E>
__global__ __launch_bounds__(256) void gather_fwd_kernel(GatherArgs a, int bh0, int64_t nrows) {
  const int TPQ = a.D / 8;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = gid / TPQ;
  if (row >= nrows) return;
  const int d0 = (int)(gid - row * TPQ) * 8;
  const int64_t bh = bh0 + row / a.L, l = row % a.L, bb = bh / a.H, h = bh - bb * a.H;
  const int64_t qh = (bb * a.L + l) * a.H + h;
  const int n = a.slot_count[qh];
  const E* v = (const E*)a.v + bb * a.vsb + h * a.vsh + d0;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int u0 = 0; u0 < n; u0 += 4) {
    float x[4][8], w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool ok = u0 + j < n;
      const int leaf = ok ? a.slot_leaf[qh * a.S + u0 + j] : 0;
      w[j] = ok ? a.slot_weight[qh * a.S + u0 + j] : 0.f;
      load8f(x[j], v + (int64_t)leaf * a.vsl);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += w[j] * x[j][i];
  }
  if (a.acc32) acc8f(a.acc32 + qh * a.D + d0, acc, a.first);
  else store8f((E*)a.out + bb * a.osb + l * a.osl + h * a.osh + d0, acc);
}

// dv[b, n, h, :] = sum over leaf n's bucket (query order) of W_u dout_l, and
// for every entry (l, u) of the bucket delta[qh, u] = dout_l . v[n] (the
// leaf's value row is loaded once; the dout rows are the ones dv reads).
// TP = D / 8 rounded up to a power of two lanes per leaf, 8 head dims each
// (lanes past D idle), so the dot products reduce with xor shuffles inside
// the group; grid (.., B*H).
template <typename E, int TP>
__global__ __launch_bounds__(256) void scatter_dv_kernel(GatherArgs a) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t n = gid / TP;
  if (n >= a.N) return;  // whole groups: TP divides the workgroup size
  const int d0 = (int)(gid - n * TP) * 8;
  const bool on = d0 < a.D;
  const int bh = blockIdx.y, bb = bh / a.H, h = bh - bb * a.H;
  const int* bs = a.block_start + (int64_t)bh * (a.N + 1);
  const int* ord = a.order + (int64_t)bh * a.L * a.S;
  const int e0 = bs[n], e1 = bs[n + 1];
  const E* g = (const E*)a.g + bb * a.gsb + h * a.gsh + (on ? d0 : 0);
  float vn[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (on) load8f(vn, (const E*)a.v + bb * a.vsb + n * a.vsl + h * a.vsh + d0);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int e = e0; e < e1; e += 4) {
    float x[4][8], w[4];
    int64_t slot[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool ok = e + j < e1;
      const int ent = ok ? ord[e + j] : 0;
      const int l = ent / a.S, u = ent - l * a.S;
      slot[j] = (((int64_t)bb * a.L + l) * a.H + h) * a.S + u;
      w[j] = ok ? a.slot_weight[slot[j]] : 0.f;
      load8f(x[j], g + (int64_t)l * a.gsl);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float dot = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        acc[i] += w[j] * x[j][i];
        dot += x[j][i] * vn[i];
      }
#pragma unroll
      for (int o = 1; o < TP; o <<= 1) dot += __shfl_xor(dot, o, 64);
      if (d0 == 0 && e + j < e1) a.delta[slot[j]] = dot;
    }
  }
  if (on) {
    if (a.acc32) acc8f(a.acc32 + ((bb * (int64_t)a.N + n) * a.H + h) * a.D + d0, acc, a.first);
    else store8f((E*)a.out + bb * a.osb + n * a.osl + h * a.osh + d0, acc);
  }
}

static GatherArgs gather_args(const Plan& P, const void* v, const char* rec) {
  GatherArgs a;
  a.L = (int)P.L;
  a.N = (int)P.N;
  a.H = (int)P.H;
  a.S = (int)P.S;
  a.D = (int)P.D;
  a.v = v;
  a.vsb = P.p.v_strides[0]; a.vsl = P.p.v_strides[1]; a.vsh = P.p.v_strides[2];
  a.g = nullptr;
  a.gsb = a.gsl = a.gsh = 0;
  a.out = nullptr;
  a.osb = a.osl = a.osh = 0;
  a.slot_leaf = (const int*)(rec + P.rec.slot_leaf);
  a.slot_weight = (const float*)(rec + P.rec.slot_weight);
  a.slot_count = (const int*)(rec + P.rec.slot_count);
  a.order = (const int*)(rec + P.rec.order);
  a.block_start = (const int*)(rec + P.rec.block_start);
  a.delta = nullptr;
  a.acc32 = nullptr;
  a.first = P.acc.first;
  return a;
}

template <typename E>
static hipError_t gather_fwd_t(const Plan& P, const void* v, void* out, const char* rec, int bh0, int nbh,
                               hipStream_t st) {
  GatherArgs a = gather_args(P, v, rec);
  a.out = out;
  a.osb = P.p.o_strides[0]; a.osl = P.p.o_strides[1]; a.osh = P.p.o_strides[2];
  a.acc32 = P.acc.out32;
  const int64_t nrows = (int64_t)nbh * P.L;
  const int64_t nthr = nrows * (P.D / 8);
  hipLaunchKernelGGL(gather_fwd_kernel<E>, dim3((unsigned)((nthr + 255) / 256)), dim3(256), 0, st, a, bh0, nrows);
  return hipGetLastError();
}

template <typename E>
static hipError_t gather_bwd_t(const Plan& P, const void* v, const void* g, void* dv, const char* rec, float* delta,
                               hipStream_t st) {
  GatherArgs a = gather_args(P, v, rec);
  a.g = g;
  a.gsb = P.p.g_strides[0]; a.gsl = P.p.g_strides[1]; a.gsh = P.p.g_strides[2];
  a.delta = delta;
  a.out = dv;
  a.osb = P.p.v_strides[0]; a.osl = P.p.v_strides[1]; a.osh = P.p.v_strides[2];
  a.acc32 = P.acc.dv32;
  const int tp = P.D <= 32 ? 4 : P.D <= 64 ? 8 : 16;
  const int64_t nthr = P.N * tp;
  const dim3 grid((unsigned)((nthr + 255) / 256), (unsigned)P.BH);
  if (tp == 4) hipLaunchKernelGGL((scatter_dv_kernel<E, 4>), grid, dim3(256), 0, st, a);
  else if (tp == 8) hipLaunchKernelGGL((scatter_dv_kernel<E, 8>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((scatter_dv_kernel<E, 16>), grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_gather_fwd(const Plan& P, const void* v, void* out, const char* rec, int bh0, int nbh,
                             hipStream_t st) {
  switch (P.p.dtype) {
    case TA_F32: return gather_fwd_t<float>(P, v, out, rec, bh0, nbh, st);
    case TA_BF16: return gather_fwd_t<bf16>(P, v, out, rec, bh0, nbh, st);
    default: return gather_fwd_t<f16>(P, v, out, rec, bh0, nbh, st);
  }
}

hipError_t launch_gather_bwd(const Plan& P, const void* v, const void* g, void* dv, const char* rec, char* ws,
                             hipStream_t st) {
  float* delta = (float*)(ws + P.bws.delta);
  switch (P.p.dtype) {
    case TA_F32: return gather_bwd_t<float>(P, v, g, dv, rec, delta, st);
    case TA_BF16: return gather_bwd_t<bf16>(P, v, g, dv, rec, delta, st);
    default: return gather_bwd_t<f16>(P, v, g, dv, rec, delta, st);
  }
}

}  // namespace ta
