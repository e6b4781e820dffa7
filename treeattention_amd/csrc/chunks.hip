// Problems with more samples than one launch takes (num_samples > 64): the
// samples are drawn and used in chunks of at most 64 (capi.cpp runs the
// chunks), and these kernels join them.
//
// The reference draws all of a query's samples at once and normalizes their
// weights with one softmax (_tree_mha.py:399, _autograd.py:692,495-498).  A
// chunk's sampler normalizes over its own samples, w^g_s = exp(l_s - lse_g),
// and records lse_g; the query's weights over all samples are then
// w_s = alpha_g w^g_s with alpha_g = exp(lse_g - lse), lse = logsumexp_g lse_g.
// Scaling the chunk's weights and its summed per-block weights by alpha_g
// before the leaf stage makes every later kernel see the weights over all
// samples, so the chunks' outputs simply add.  In the backward the per-sample
// gradient dl_s = w_s (dout . o_s - dout . out) needs dout . out over all
// samples, which chunk_mean_kernel computes once from the forward's float
// output.
#include "launch.h"

namespace ta {

// One thread per (batch, position, head, sample): the sample's chunk g scales
// its weight and (if the sample's index is below the chunk's distinct-block
// count) one summed block weight of the chunk by alpha_g, and copies its leaf
// block into the (B, L, H, S) array of all samples.
__global__ __launch_bounds__(256) void chunk_merge_kernel(ChunkRecs R, float* __restrict__ weights, int64_t wsb,
                                                          int64_t wsl, int64_t wsh, int* __restrict__ leaf_all,
                                                          int L, int H, int S, int64_t nqh) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t qh = gid / S;
  if (qh >= nqh) return;
  const int s = (int)(gid - qh * S);
  float mx = -__builtin_inff();
  for (int g = 0; g < R.n; ++g) mx = fmaxf(mx, R.lse[g][qh]);
  float tot = 0.f;
  for (int g = 0; g < R.n; ++g) tot += expf(R.lse[g][qh] - mx);
  const float lse = mx + logf(tot);
  int g = 0;
  while (g + 1 < R.n && s >= R.s0[g + 1]) ++g;
  const float alpha = expf(R.lse[g][qh] - lse);
  const int u = s - R.s0[g];
  const int64_t h = qh % H, bl = qh / H, l = bl % L, bb = bl / L;
  weights[bb * wsb + l * wsl + h * wsh + s] *= alpha;
  if (u < R.slot_count[g][qh]) R.slot_weight[g][qh * R.S[g] + u] *= alpha;
  leaf_all[qh * S + s] = R.leaf[g][qh * R.S[g] + u];
}

hipError_t launch_chunk_merge(const Plan& P, const ChunkRecs& R, float* weights, int* leaf_all, hipStream_t st) {
  const int64_t nqh = P.B * P.L * P.H;
  const int S = (int)P.s_total;
  const int64_t n = nqh * S;
  hipLaunchKernelGGL(chunk_merge_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, R, weights,
                     P.p.w_strides[0], P.p.w_strides[1], P.p.w_strides[2], leaf_all, (int)P.L, (int)P.H, S, nqh);
  return hipGetLastError();
}

// mean[b, l, h] = dout[b, l, h, :] . out[b, l, h, :] (out: the forward's
// (B, L, H, D) rows, float or E); a group of DG lanes per row (DG = D / 8
// rounded up to a power of two), eight dims per lane in 16-byte loads, then a
// butterfly over the group (a fixed order).
template <typename E, typename O, int DG>
__global__ __launch_bounds__(256) void chunk_mean_kernel(const E* __restrict__ g, int64_t gsb, int64_t gsl,
                                                         int64_t gsh, const O* __restrict__ out,
                                                         float* __restrict__ mean, int L, int H, int D, int64_t nqh) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t qh = gid / DG;
  const int dg = (int)(gid - qh * DG);
  float s = 0.f;
  if (qh < nqh && 8 * dg < D) {
    const int64_t h = qh % H, bl = qh / H, l = bl % L, bb = bl / L;
    float gv[8], ov[8];
    ld8f(gv, g + bb * gsb + l * gsl + h * gsh + 8 * dg);
    ld8f(ov, out + qh * D + 8 * dg);
#pragma unroll
    for (int i = 0; i < 8; ++i) s += gv[i] * ov[i];
  }
#pragma unroll
  for (int m = 1; m < DG; m <<= 1) s += __shfl_xor(s, m, 64);
  if (qh < nqh && dg == 0) mean[qh] = s;
}

template <typename E, typename O, int DG>
static void mean_launch(const Plan& P, const void* g, const O* out, float* mean, hipStream_t st) {
  const int64_t nqh = P.B * P.L * P.H;
  const dim3 grid((unsigned)((nqh * DG + 255) / 256));
  const int64_t* gs = P.p.g_strides;
  hipLaunchKernelGGL((chunk_mean_kernel<E, O, DG>), grid, dim3(256), 0, st, (const E*)g, gs[0], gs[1], gs[2], out,
                     mean, (int)P.L, (int)P.H, (int)P.D, nqh);
}

template <typename E>
static void mean_d(const Plan& P, const void* g, const void* out, bool out_e, float* mean, hipStream_t st) {
  if (out_e) {
    if (P.D <= 32) mean_launch<E, E, 4>(P, g, (const E*)out, mean, st);
    else if (P.D <= 64) mean_launch<E, E, 8>(P, g, (const E*)out, mean, st);
    else mean_launch<E, E, 16>(P, g, (const E*)out, mean, st);
  } else {
    if (P.D <= 32) mean_launch<E, float, 4>(P, g, (const float*)out, mean, st);
    else if (P.D <= 64) mean_launch<E, float, 8>(P, g, (const float*)out, mean, st);
    else mean_launch<E, float, 16>(P, g, (const float*)out, mean, st);
  }
}

hipError_t launch_chunk_mean(const Plan& P, const void* g, const void* out, bool out_e, float* mean, hipStream_t st) {
  switch (P.p.dtype) {
    case TA_F32: mean_d<float>(P, g, out, out_e, mean, st); break;
    case TA_BF16: mean_d<bf16>(P, g, out, out_e, mean, st); break;
    default: mean_d<f16>(P, g, out, out_e, mean, st);
  }
  return hipGetLastError();
}

// dst[b, r, h, :] (E, strided) = src[((b R + r) H + h) D + :] (float); one
// thread per 8 elements of a row (D a multiple of 8).
template <typename E>
__global__ __launch_bounds__(256) void cast_rows_kernel(const float* __restrict__ src, E* __restrict__ dst,
                                                        int64_t sb, int64_t sr, int64_t sh, int R, int H, int D,
                                                        int64_t n8) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n8) return;
  const int64_t row = e / (D / 8);
  const int d0 = (int)(e - row * (D / 8)) * 8;
  const int64_t h = row % H, br = row / H, r = br % R, bb = br / R;
  const float4 x = *(const float4*)(src + row * D + d0), y = *(const float4*)(src + row * D + d0 + 4);
  E* o = dst + bb * sb + r * sr + h * sh + d0;
  if constexpr (sizeof(E) == 2) {
    typedef __attribute__((ext_vector_type(8))) E e8;
    e8 v;
    v[0] = (E)x.x; v[1] = (E)x.y; v[2] = (E)x.z; v[3] = (E)x.w;
    v[4] = (E)y.x; v[5] = (E)y.y; v[6] = (E)y.z; v[7] = (E)y.w;
    *(e8*)o = v;
  } else {
    *(float4*)o = x;
    *(float4*)(o + 4) = y;
  }
}

hipError_t launch_cast_rows(int dtype, const float* src, void* dst, const int64_t* st3, int64_t B, int64_t R,
                            int64_t H, int64_t D, hipStream_t st) {
  const int64_t n8 = B * R * H * (D / 8);
  const dim3 grid((unsigned)((n8 + 255) / 256));
  switch (dtype) {
    case TA_F32:
      hipLaunchKernelGGL(cast_rows_kernel<float>, grid, dim3(256), 0, st, src, (float*)dst, st3[0], st3[1], st3[2],
                         (int)R, (int)H, (int)D, n8);
      break;
    case TA_BF16:
      hipLaunchKernelGGL(cast_rows_kernel<bf16>, grid, dim3(256), 0, st, src, (bf16*)dst, st3[0], st3[1], st3[2],
                         (int)R, (int)H, (int)D, n8);
      break;
    default:
      hipLaunchKernelGGL(cast_rows_kernel<f16>, grid, dim3(256), 0, st, src, (f16*)dst, st3[0], st3[1], st3[2],
                         (int)R, (int)H, (int)D, n8);
  }
  return hipGetLastError();
}

}  // namespace ta
