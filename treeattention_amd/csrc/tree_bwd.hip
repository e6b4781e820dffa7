// K4b: tree part of the backward (the reference's per-depth grad_logit and
// q/k accumulation, _autograd.py:789-856 and
// accumulate_qk_non_causal_all_depths_prepared.cu:104-161), deterministic.
//
// Per sample s, dlogp_s = w_s (delta_s - sum_s' w_s' delta_s') (softmax over
// samples, _autograd.py:791-794).  Samples that picked the same leaf block u
// share their whole path, so only the per-block sum matters:
//   dl_u = sum_{s->u} dlogp_s = W_u (delta_u - sum_u' W_u' delta_u'),
// W_u the summed sample weight.  At depth d, node n with child logits x_j and
// probabilities p_j receives, for every child j,
//   G[n, j] = sum_{u under child j} dl_u  -  p_j * sum_{u under n} dl_u
// (zero where the logit was clamped).  A query's distinct blocks are sorted,
// so the blocks under any node are one contiguous run, summed by segmented
// scans with one writer per entry of G -- no conflicts, no atomics.  Then
//   tree_dq_kernel: dq = sum_u dq_pair[u] + sum_chunks G C_chunk (MFMA); it
//     also writes G^T and Q^T per tile of 64 queries, queries contiguous
//     (one contiguous block per tile and chunk);
//   tree_dc_kernel: dC = G^T Q per query split, a plain MFMA product of the
//     two (no recomputation of logits or G), skipping under exact causal
//     masking the (row tile, query block) pairs whose G^T rows are all zero;
//   dsum_reduce_kernel adds the splits in order;
//   pool_adjoint_kernel: dk = dk_leaf + (summaries map)^T dC, which for
//   compat summaries is the transpose of the reference's Haar keys
//   (_treeattn_common.py:70-86).
// The causal correction adds the same -log A_root to every sample of a
// query; since sum_s dlogp_s = 0 it has no gradient.
#include <type_traits>

#include "launch.h"

namespace ta {

// Child-summary columns per MFMA logit chunk of tree_dq_kernel: 64 at head
// dims up to 64 (the query tile's LDS then leaves room for three workgroups
// per CU; measured 19 % faster at D = 32 and 64), 128 above (where the
// registers allow two workgroups per CU either way and more chunks cost more
// barriers).  The logit tile's row stride is CH + 4 floats, G's CH + 8 elements.
constexpr int chunk_cols(int D) { return D <= 64 ? 64 : 128; }

struct TreeArgs {
  Geo geo;
  int L, N, H, S, D, causal, mode;
  float maxhalf;
  const void* q;
  int64_t qsb, qsl, qsh;
  const void* sum_hi;  // E (BH, NS, D) (float inputs: the float summaries)
  const void* sum_t;   // E (BH, D, NS)
  const int* slot_leaf;
  const int* slot_count;
  const float* slot_weight;
  const float* delta;
  const void* dq_part;
  float* dl;           // (B, L, H, S) per distinct block
  void* gt;            // E (BH, Lp / 64, NS, 64): G^T per query tile
  void* qt;            // E (BH, Lp / 64, D, 64): Q^T per query tile
  int64_t Lp;
  void* dq;
  float* dsum_part;
  float* dsum;
  const float* dk_leaf;
  void* dk;
  int64_t ksb, ksl, ksh;
  int qsplit;
  int BHn;  // B * H
  // reference causal mode
  int refc, t0;           // t0: first sampled query row (queries below it are the exact head)
  int64_t nqh;            // B * L * H
  const float* sum32;     // float (BH, NS, D) summaries
  const int* dstar;       // (L) first uncorrected depth per query
  float* rc_coef;         // (B, L, H, T)
  float* rc_rho;          // (B, L, H, T)
  float* rc_g;            // (B, L, H, T): the boundary children's gradient g (left +g, right -g) per depth
  // levels d < Tb are dense (G tiles; G^T rows 0 .. nsd - 1 per query tile); deeper ones
  // are the band kernels' (tree_band_kernel)
  int Tb, nsd;
  int dqp;  // 1: add each query's per-pair dq rows (leaf dq and deep-level tree dq)
  int dkl;  // 1: add the leaf part of dk
  // a chunk of a problem with many samples: dq goes to float rows (written by
  // the first chunk, added by later ones), and so does the summary gradient
  float* dq32;
  int first;
  const float* dcp;  // path rows: (BH, NL, T*b, D) per leaf block
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

// dl_u = W_u (delta_u - sum_u' W_u' delta_u').  Lane group of P lanes (P =
// S rounded up to a power of two) per (b, l, h); butterfly sum in the group.
// A chunk of a problem with many samples passes the sum over all its samples
// (dout . out) as `mean` (its W are the weights over all samples).
__global__ __launch_bounds__(256) void slot_dlogp_kernel(const int* __restrict__ slot_count,
                                                         const float* __restrict__ slot_weight,
                                                         const float* __restrict__ delta, float* __restrict__ dl,
                                                         int S, int P, int64_t nqh, const float* __restrict__ mean) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t qh = gid / P;
  const int u = (int)(gid - qh * P);
  const bool in = qh < nqh;
  const int n = in ? slot_count[qh] : 0;
  const bool act = u < n;
  const float w = act ? slot_weight[qh * S + u] : 0.f;
  const float dt = act ? delta[qh * S + u] : 0.f;
  float tot = w * dt;
  if (mean) {
    tot = in ? mean[qh] : 0.f;
  } else {
    for (int o = 1; o < P; o <<= 1) tot += __shfl_xor(tot, o, 64);
  }
  if (act) dl[qh * S + u] = w * (dt - tot);
}

// Reference causal mode (_tree_mha.py:198-262): a sampled query row t whose
// lanes were not all on the boundary path from depth D* on (D* < T) gives the
// samples still on the path at D* the log-mass M_{D*} in their log-prob, and
// M_{D*} depends on the boundary logits of depths d >= D*:
//   M_d = logsumexp(M_{d+1} + logsig(on_d), m_off,d + logsig(off_d)),  M_T = 0,
//   dM_{D*}/dx_j(d) = Gamma_d (rho_j - p_j),   Gamma_d = prod_{D* <= e < d} pi_e,
// with p the child probabilities of boundary node d, rho_on = pi_d =
// exp(M_{d+1} + logsig(on_d) - M_d), rho_off = 1 - pi_d.  One thread per
// (batch, position, head) writes coef_d = A_on Gamma_d (A_on = the summed dl
// of the slots below the depth-D* boundary node) and rho_d = pi_d for
// d >= D*, zeros elsewhere; tree_dq adds coef_d (rho_j - p_j) to G.  The
// common -M_0 of every sample of a row has no gradient (sum_s dlogp_s = 0).
template <typename E>
__global__ __launch_bounds__(256) void ref_causal_grad_kernel(TreeArgs a) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int H = a.H, L = a.L, T = a.geo.T, D = a.D;
  if (gid >= a.nqh) return;
  const int h = (int)(gid % H);
  const int64_t bl = gid / H;
  const int t = (int)(bl % L), bb = (int)(bl / L);
  float* cf = a.rc_coef + gid * T;
  float* rh = a.rc_rho + gid * T;
  float* gg = a.rc_g + gid * T;
  for (int d = 0; d < T; ++d) {
    cf[d] = 0.f;
    rh[d] = 0.f;
    gg[d] = 0.f;
  }
  if (t < a.t0) return;
  const int ds = a.dstar[t];
  if (ds >= T) return;
  const int c = t, bh = bb * H + h;
  const E* qr = (const E*)a.q + bb * a.qsb + (int64_t)t * a.qsl + h * a.qsh;
  // bottom-up masses and pi_d for d = T-1 .. D*
  float m = 0.f;
  for (int d = T - 1; d >= ds; --d) {
    const float* crow = a.sum32 + ((int64_t)bh * a.geo.NS + a.geo.off[d + 1] + 2 * (c >> (T - d))) * D;
    const float x = 2.f * dot_row(qr, crow, D);
    const int dir = (c >> (T - 1 - d)) & 1;
    const float on = dir ? logsig(-x) : logsig(x), off = dir ? logsig(x) : logsig(-x);
    const float a0 = m + on;
    float md = a0;
    if (dir) {
      const float a1 = logf((float)(1 << (T - 1 - d))) + off;
      const float mx = fmaxf(a0, a1);
      md = mx + logf(expf(a0 - mx) + expf(a1 - mx));
    }
    rh[d] = expf(a0 - md);
    m = md;
  }
  // A_on: slots below the depth-D* boundary node
  const int node = c >> (T - ds);
  const int cnt = a.slot_count[gid];
  float A = 0.f;
  for (int u = 0; u < cnt; ++u)
    if ((a.slot_leaf[gid * a.S + u] >> (T - ds)) == node) A += a.dl[gid * a.S + u];
  float gam = 1.f;
  for (int d = ds; d < T; ++d) {
    cf[d] = A * gam;
    gam *= rh[d];
  }
  // the gradient of the boundary node's left child logit at depth d,
  // g = coef_d (rho_left - p_left) (the right child gets -g); the dense
  // levels add it to G in tree_dq_kernel, the band levels through rc_g
  for (int d = max(ds, a.Tb); d < T; ++d) {
    const float* crow = a.sum32 + ((int64_t)bh * a.geo.NS + a.geo.off[d + 1] + 2 * (c >> (T - d))) * D;
    const float pl = 1.f / (1.f + __expf(-2.f * dot_row(qr, crow, D)));
    const float rl = ((c >> (T - 1 - d)) & 1) ? 1.f - rh[d] : rh[d];
    gg[d] = cf[d] * (rl - pl);
  }
}

// Query tile of the dq kernel in LDS: child logits of the current chunk, G of
// the chunk, and each query's distinct leaf blocks, their dl and count.
template <typename E>
struct TileSmem {
  float* Xs;   // [64][chunk columns + 4]
  E* Gm;       // [64][chunk columns + 8]
  int* lf;     // [64][S]
  float* dls;  // [64][S]
  int* cn;     // [64]
  float* scv;  // [64 * P][2] per scan lane of a level: A_row, A_n (P = 8 or 16 lanes per query)
  int* sci;    // [64 * P][3] per scan lane: child row, node, run-end flags | children mask << 8
};

template <typename E>
__device__ __forceinline__ void load_slots(const TreeArgs& a, const TileSmem<E>& sm, int bb, int h, int l0, int nq,
                                           int tid) {
  const int S = a.S;
  const int64_t qh0 = ((int64_t)bb * a.L + l0) * a.H + h;
  for (int e = tid; e < kQueryTile * S; e += 256) {
    const int qi = e / S, u = e - qi * S;
    const int64_t o = (qh0 + (int64_t)qi * a.H) * S + u;
    sm.lf[e] = qi < nq ? a.slot_leaf[o] : 0;
    sm.dls[e] = qi < nq ? a.dl[o] : 0.f;
  }
  if (tid < kQueryTile) sm.cn[tid] = tid < nq ? a.slot_count[qh0 + (int64_t)tid * a.H] : 0;
}

// Lane (i - O) of the same 16-lane row (0 past the row start): a DPP row_shr,
// a register move without an LDS round trip.  row_shl by one likewise.
template <int O>
__device__ __forceinline__ int row_shr(int x) {
  return __builtin_amdgcn_update_dpp(0, x, 0x110 + O, 0xf, 0xf, true);
}
template <int O>
__device__ __forceinline__ float row_shr(float x) {
  return __builtin_bit_cast(float, row_shr<O>(__builtin_bit_cast(int, x)));
}
__device__ __forceinline__ int row_shl1(int x) { return __builtin_amdgcn_update_dpp(0, x, 0x101, 0xf, 0xf, true); }

// x from lane u - O of this lane's group of P lanes (the caller masks u < O)
template <int P, int O, typename T>
__device__ __forceinline__ T grp_up(T x) {
  if constexpr (P <= 16) return row_shr<O>(x);
  else return __shfl_up(x, O, P);
}
template <int P>
__device__ __forceinline__ int grp_down1(int x) {
  if constexpr (P <= 16) return row_shl1(x);
  else return __shfl_down(x, 1, P);
}

// build_g_p in two halves for levels wider than one chunk (P <= 16, b = 2 or
// 4): build_g_scan runs the segmented scans of depth d once and keeps each
// lane's sums and run flags in LDS; build_g_emit then writes each chunk's
// entries from them.  Every lane reads back only what it wrote itself.
template <typename E, int P, int kB>
__device__ __forceinline__ void build_g_scan(const Geo& G, int d, int S, int nq, const int* lf, const float* dls,
                                             const int* cn, float* scv, int* sci, int tid) {
  static_assert(P <= 16 && (kB == 2 || kB == 4), "hoisted scans: P <= 16, b = 2 or 4");
  constexpr int LP = P <= 1 ? 0 : P <= 2 ? 1 : P <= 4 ? 2 : P <= 8 ? 3 : 4;
  constexpr int lb = kB == 2 ? 1 : 2;
  const int sh = lb * (G.T - d), sh2 = sh - lb;
  const int lane = tid & 63;
  for (int e0 = 0; e0 < (kQueryTile << LP); e0 += 256) {
    const int e = e0 + tid;
    const int qi = e >> LP, u = e & (P - 1);
    const int cnt = qi < nq ? cn[qi] : 0;
    const bool act = u < cnt;
    const int leaf = act ? lf[qi * S + u] : 0;
    const float dl = act ? dls[qi * S + u] : 0.f;
    const int crow = act ? (leaf >> sh2) : -1 - u;
    const int node = act ? (leaf >> sh) : -1 - u;
    float vc = dl, vn = dl;
    int has0 = act ? 1 << (crow & (kB - 1)) : 0;
    auto step = [&](auto oc) {
      constexpr int O = decltype(oc)::value;
      if constexpr (O < P) {
        const float tc = grp_up<P, O>(vc);
        const float tn = grp_up<P, O>(vn);
        const int kc = grp_up<P, O>(crow);
        const int kn = grp_up<P, O>(node);
        const int h0 = grp_up<P, O>(has0);
        if (u >= O) {
          if (kc == crow) vc += tc;
          if (kn == node) {
            vn += tn;
            has0 |= h0;
          }
        }
      }
    };
    step(std::integral_constant<int, 1>());
    step(std::integral_constant<int, 2>());
    step(std::integral_constant<int, 4>());
    step(std::integral_constant<int, 8>());
    const int nxc = grp_down1<P>(crow);
    const int nxn = grp_down1<P>(node);
    const bool last = u + 1 >= cnt;
    const bool cend = act && (last || nxc != crow);
    const bool nend = act && (last || nxn != node);
    const uint64_t rest = __ballot(nend) >> lane;
    const int src = rest ? lane + __builtin_ctzll(rest) : lane;
    const float An = __shfl(vn, src, 64);
    scv[2 * e] = vc;
    scv[2 * e + 1] = An;
    sci[3 * e] = crow;
    sci[3 * e + 1] = node;
    sci[3 * e + 2] = (cend ? 1 : 0) | (nend ? 2 : 0) | (has0 << 8);
  }
}

template <typename E, int P, int kB, int kXS, int kGS>
__device__ __forceinline__ void build_g_emit(const Geo& G, int c0, int ncols, float maxhalf, const float* Xs,
                                             const float* scv, const int* sci, E* Gm, int tid) {
  constexpr int LP = P <= 1 ? 0 : P <= 2 ? 1 : P <= 4 ? 2 : P <= 8 ? 3 : 4;
  constexpr int lb = kB == 2 ? 1 : 2;
  for (int e0 = 0; e0 < (kQueryTile << LP); e0 += 256) {
    const int e = e0 + tid;
    const int qi = e >> LP;
    const int fl = sci[3 * e + 2];
    const bool cend = fl & 1, nend = fl & 2;
    const int node = sci[3 * e + 1];
    const int base = (node << lb) - c0;
    if ((cend || nend) && base >= 0 && base < ncols) {
      const int crow = sci[3 * e], has0 = fl >> 8;
      const float vc = scv[2 * e], An = scv[2 * e + 1];
      const float* xr = Xs + qi * kXS + base;
      E* gr = Gm + qi * kGS + base;
      float xv[kB], ev[kB];
      if constexpr (kB == 4) {
        const float4 t = *(const float4*)xr;
        xv[0] = t.x; xv[1] = t.y; xv[2] = t.z; xv[3] = t.w;
      } else {
        const float2 t = *(const float2*)xr;
        xv[0] = t.x; xv[1] = t.y;
      }
      float mx = -__builtin_inff();
#pragma unroll
      for (int j = 0; j < kB; ++j) mx = fmaxf(mx, clamp_h(xv[j], maxhalf));
      float se = 0.f;
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        ev[j] = __expf(clamp_h(xv[j], maxhalf) - mx);
        se += ev[j];
      }
      const float pa = An / se;
      const int jc = crow & (kB - 1);
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        const bool live = xv[j] >= -maxhalf && xv[j] <= maxhalf;
        if (cend && j == jc) gr[j] = (E)(live ? vc - ev[j] * pa : 0.f);
        else if (nend && !((has0 >> j) & 1)) gr[j] = (E)(live ? -ev[j] * pa : 0.f);
      }
    }
  }
}

// G for depth d, chunk [c0, c0 + ncols) of the level's child rows, into
// Gm[q][col].  A group of P >= S lanes per query, lane u = slot u (slots
// ascend by leaf block, so the slots under one child row form a run, and so
// do the slots under one node).  Segmented inclusive scans over the runs give
// A_row (sum of dl under the child row) and A_n (under the node); for P <= 16
// the scan steps are DPP row shifts.  The last lane of each child run writes
// G[n, j] = A_row - p_j A_n; the last lane of each node run writes -p_j A_n
// for the node's children without sampled blocks.  Every entry has one
// writer and every sum a fixed order: deterministic, no atomics.  Clamped
// logits get 0.
// kB: the branching factor when known at compile time (2 or 4), else 0.
template <typename E, int P, int kB, int kXS, int kGS>
__device__ __forceinline__ void build_g_p(const Geo& G, int d, int c0, int ncols, int S, int nq, float maxhalf,
                                          const float* Xs, const int* lf, const float* dls, const int* cn, E* Gm,
                                          int tid) {
  constexpr int LP = P <= 1 ? 0 : P <= 2 ? 1 : P <= 4 ? 2 : P <= 8 ? 3 : P <= 16 ? 4 : P <= 32 ? 5 : 6;
  const int b = kB > 0 ? kB : G.b, lb = kB == 2 ? 1 : kB == 4 ? 2 : G.lb;
  const int sh = lb * (G.T - d), sh2 = sh - lb;
  const int lane = tid & 63;
  for (int e0 = 0; e0 < (kQueryTile << LP); e0 += 256) {
    const int e = e0 + tid;
    const int qi = e >> LP, u = e & (P - 1);
    const int cnt = qi < nq ? cn[qi] : 0;
    const bool act = u < cnt;
    const int leaf = act ? lf[qi * S + u] : 0;
    const float dl = act ? dls[qi * S + u] : 0.f;
    const int crow = act ? (leaf >> sh2) : -1 - u;  // inactive lanes: singleton runs
    const int node = act ? (leaf >> sh) : -1 - u;
    float vc = dl, vn = dl;
    // children of the node with sampled blocks (b <= 64: two 32-bit words)
    int has0 = 0, has1 = 0;
    if (act) {
      const int j = crow & (b - 1);
      if (j < 32) has0 = 1 << j;
      else has1 = 1 << (j - 32);
    }
    auto step = [&](auto oc) {
      constexpr int O = decltype(oc)::value;
      if constexpr (O < P) {
        const float tc = grp_up<P, O>(vc);
        const float tn = grp_up<P, O>(vn);
        const int kc = grp_up<P, O>(crow);
        const int kn = grp_up<P, O>(node);
        const int h0 = grp_up<P, O>(has0);
        const int h1 = kB > 0 ? 0 : grp_up<P, O>(has1);  // b <= 32: has1 stays 0
        if (u >= O) {
          if (kc == crow) vc += tc;
          if (kn == node) {
            vn += tn;
            has0 |= h0;
            has1 |= h1;
          }
        }
      }
    };
    step(std::integral_constant<int, 1>());
    step(std::integral_constant<int, 2>());
    step(std::integral_constant<int, 4>());
    step(std::integral_constant<int, 8>());
    step(std::integral_constant<int, 16>());
    step(std::integral_constant<int, 32>());
    const int nxc = grp_down1<P>(crow);
    const int nxn = grp_down1<P>(node);
    const bool last = u + 1 >= cnt;
    const bool cend = act && (last || nxc != crow);
    const bool nend = act && (last || nxn != node);
    const uint64_t rest = __ballot(nend) >> lane;
    const int src = rest ? lane + __builtin_ctzll(rest) : lane;
    const float An = __shfl(vn, src, 64);
    const int base = (node << lb) - c0;
    if ((cend || nend) && base >= 0 && base < ncols) {
      const float* xr = Xs + qi * kXS + base;
      E* gr = Gm + qi * kGS + base;
      if constexpr (kB > 0) {
        // the node's kB logits in one LDS read (base is a multiple of kB)
        float xv[kB], ev[kB];
        if constexpr (kB == 4) {
          const float4 t = *(const float4*)xr;
          xv[0] = t.x; xv[1] = t.y; xv[2] = t.z; xv[3] = t.w;
        } else {
          const float2 t = *(const float2*)xr;
          xv[0] = t.x; xv[1] = t.y;
        }
        float mx = -__builtin_inff();
#pragma unroll
        for (int j = 0; j < kB; ++j) mx = fmaxf(mx, clamp_h(xv[j], maxhalf));
        float se = 0.f;
#pragma unroll
        for (int j = 0; j < kB; ++j) {
          ev[j] = __expf(clamp_h(xv[j], maxhalf) - mx);
          se += ev[j];
        }
        const float pa = An / se;  // p_j A_n = ev[j] * pa
        const int jc = crow & (kB - 1);
#pragma unroll
        for (int j = 0; j < kB; ++j) {
          const bool live = xv[j] >= -maxhalf && xv[j] <= maxhalf;
          if (cend && j == jc) gr[j] = (E)(live ? vc - ev[j] * pa : 0.f);
          else if (nend && !((has0 >> j) & 1)) gr[j] = (E)(live ? -ev[j] * pa : 0.f);
        }
      } else {
        float mx = -__builtin_inff();
        for (int j = 0; j < b; ++j) mx = fmaxf(mx, clamp_h(xr[j], maxhalf));
        float se = 0.f;
        for (int j = 0; j < b; ++j) se += __expf(clamp_h(xr[j], maxhalf) - mx);
        const float lse = mx + __logf(se);
        if (cend) {
          const int j = crow & (b - 1);
          const float x = xr[j];
          const bool live = x >= -maxhalf && x <= maxhalf;
          gr[j] = (E)(live ? vc - __expf(clamp_h(x, maxhalf) - lse) * An : 0.f);
        }
        if (nend) {
          for (int j = 0; j < b; ++j) {
            if (j < 32 ? ((has0 >> j) & 1) : ((has1 >> (j - 32)) & 1)) continue;
            const float x = xr[j];
            const bool live = x >= -maxhalf && x <= maxhalf;
            gr[j] = (E)(live ? -__expf(clamp_h(x, maxhalf) - lse) * An : 0.f);
          }
        }
      }
    }
  }
}

// One workgroup per 64 queries of one (batch, head).  All 64 query rows are
// held by every wave as MFMA fragments.  Per chunk of a level's child rows:
//   X^T = C_chunk Q^T   (wave w: column tiles w, w+4, ...; C rows from global)
//   G   = build_g(X)    (LDS)
//   dq^T += C_chunk^T G^T (wave w: head-dim tiles w, w+4, ...)
// and G^T goes to global for the summary-gradient product.  The epilogue adds
// the leaf parts dq_pair of each query's distinct blocks.
// kP: lanes per query in build_g (8: S <= 8, 16: S <= 16, DPP scans; 64: shuffles).
// kB: the branching factor when known at compile time (2 or 4), else 0.
template <typename E, int D, int kP, int kB>
__global__ __launch_bounds__(256, 2) void tree_dq_kernel(TreeArgs a) {
  using M = Mfma<E>;
  using F = typename M::frag;
  constexpr int KS = D / M::K;
  constexpr int NMD = (D / 16 + 3) / 4;  // head-dim tiles per wave
  constexpr int kChunk = chunk_cols(D), kXS = kChunk + 4, kGS = kChunk + 8;
  constexpr int kSL = kP <= 8 ? 8 : 16;  // hoisted scan lanes per query
  extern __shared__ __align__(16) char smem[];
  const Geo& G = a.geo;
  const int bh = blockIdx.y, bb = bh / a.H, h = bh - bb * a.H;
  const int l0 = blockIdx.x * kQueryTile;
  const int nq = min(kQueryTile, a.L - l0);
  const int S = a.S, T = G.T;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, col = lane & 15, g = lane >> 4;
  const int64_t rows = G.NS;

  TileSmem<E> sm;
  sm.Xs = (float*)smem;
  sm.Gm = (E*)(sm.Xs + kQueryTile * kXS);
  sm.lf = (int*)(sm.Gm + kQueryTile * kGS);
  sm.dls = (float*)(sm.lf + kQueryTile * S);
  sm.cn = (int*)(sm.dls + kQueryTile * S);
  sm.scv = (float*)(sm.cn + kQueryTile);
  sm.sci = (int*)(sm.scv + 2 * kQueryTile * kSL);

  RowFrags<E, D> qa[4];
#pragma unroll
  for (int qt = 0; qt < 4; ++qt) {
    const int r = 16 * qt + col;
    qa[qt].load(r < nq ? (const E*)a.q + bb * a.qsb + (int64_t)(l0 + r) * a.qsl + h * a.qsh : nullptr, g);
  }
  load_slots<E>(a, sm, bb, h, l0, nq, tid);
  // Q^T for the summary-gradient product (rows past nq are zero fragments),
  // transposed through LDS so every global store is a 16-byte row piece
  {
    E* qst = (E*)sm.Xs;  // [D][64]
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) {
      if (qt != w) continue;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if constexpr (M::KPL == 1) {
          qst[(ks * M::K + g) * kQueryTile + 16 * qt + col] = qa[qt].f[ks];
        } else {
#pragma unroll
          for (int i = 0; i < M::KPL; ++i) qst[(ks * M::K + M::KPL * g + i) * kQueryTile + 16 * qt + col] = qa[qt].f[ks][i];
        }
      }
    }
    __syncthreads();
    E* qt_out = (E*)a.qt + ((int64_t)bh * gridDim.x + blockIdx.x) * D * kQueryTile;  // this tile's [D][64]
    for (int e = tid; e < D * (kQueryTile / 8); e += 256) {
      const int dd = e >> 3, q0 = (e & 7) * 8;
      cp8(qt_out + dd * kQueryTile + q0, qst + dd * kQueryTile + q0);
    }
    __syncthreads();
  }

  f32x4 dacc[NMD][4];
#pragma unroll
  for (int i = 0; i < NMD; ++i)
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) dacc[i][qt] = zero4();
  const E* sum_hi = (const E*)a.sum_hi;
  const E* sum_t = (const E*)a.sum_t;

  // Chunks (level d + 1, children [c0, c0 + kChunk)) in order.  Each wave
  // holds the summary fragments of its logit tiles (tiles w, w + 4 of the
  // chunk) and of its C^T rows (head-dim tiles w + 4i) for the whole chunk;
  // the next chunk's are loaded as soon as the current ones are consumed, so
  // their latency hides behind build_g and the other products.
  constexpr int KT = kChunk / M::K;  // k-steps of the C^T G^T product per chunk
  F af[2][KS];
  F at[NMD][KT];
  // Exact causal restriction: every sampled block is <= blk_hi, so only
  // children of depth-d nodes over those blocks hold G entries for this tile;
  // the products skip the other columns, and their G^T rows past the reach
  // (rounded up to 32) are not written: tree_dc_kernel skips them by the same
  // rule.  (The reference causal mode samples past the query's position.)
  const bool cz = a.causal;
  const int blk_hi = (l0 + nq - 1 + (a.N - a.L)) / G.LB;
  auto reach = [&](int d) {
    const int n = G.pw[d + 1];
    return cz ? min(n, ((blk_hi >> (G.lb * (T - d))) + 1) << G.lb) : n;
  };
  auto kcols_of = [&](int d, int c0) { return (max(0, min(kChunk, reach(d) - c0)) + 31) / 32 * 32; };
  auto load_af = [&](int d, int c0) {
    const int64_t r0 = (int64_t)bh * rows + G.off[d + 1] + c0;
    const int kc = kcols_of(d, c0);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int ct = w + 4 * j;
      if (ct < kc / 16) {
        const E* ar = sum_hi + (r0 + 16 * ct + col) * D + M::KPL * g;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) af[j][ks] = ld_frag(ar + ks * M::K);
      }
    }
  };
  auto load_at = [&](int d, int c0) {
    const int kc = kcols_of(d, c0);
#pragma unroll
    for (int i = 0; i < NMD; ++i) {
      const int md = w + 4 * i;
      if (md < D / 16) {
        const E* ap = sum_t + ((int64_t)bh * D + 16 * md + col) * rows + G.off[d + 1] + c0 + M::KPL * g;
#pragma unroll
        for (int ks = 0; ks < KT; ++ks)
          if (ks < kc / M::K) at[i][ks] = ld_frag(ap + ks * M::K);
      }
    }
  };
  const int Tb = a.Tb;  // dense depths 0 .. Tb - 1
  int d = 0, c0 = 0;
  if (Tb > 0) {
    load_af(0, 0);
    load_at(0, 0);
  }
  while (d < Tb) {
    const int lam = d + 1, lvl = G.pw[lam];
    const int ncols = min(kChunk, lvl - c0);
    const int rcols = max(0, min(ncols, reach(d) - c0));  // columns that can be nonzero
    const int rk = (rcols + 31) / 32 * 32;  // inside the level's zero padding
    int nd = d, nc0 = c0 + kChunk;
    if (nc0 >= lvl) {
      nc0 = 0;
      ++nd;
    }
    // X^T tiles: rows of C (this wave's column tiles) against all 64 queries
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int ct = w + 4 * j;
      if (ct < rk / 16) {
#pragma unroll
        for (int qt = 0; qt < 4; ++qt) {
          f32x4 c = zero4();
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) c = M::mma(af[j][ks], qa[qt].f[ks], c);
          *(f32x4*)(sm.Xs + (16 * qt + col) * kXS + 16 * ct + 4 * g) = c;
        }
      }
    }
    // this chunk's C^T fragments are complete by now (the logit MFMAs above
    // waited for every earlier load); pin them before the next chunk's loads
    // go out, so the dq product below waits for neither those loads nor the
    // G^T stores (vmcnt counts both)
#pragma unroll
    for (int i = 0; i < NMD; ++i)
#pragma unroll
      for (int ks = 0; ks < KT; ++ks) asm volatile("" ::"v"(at[i][ks]) : "memory");
    if (nd < Tb) load_af(nd, nc0);
    for (int e = tid; e < kQueryTile * rk / 8; e += 256) {
      const int r = e / (rk / 8), cc = (e - r * (rk / 8)) * 8;
      z8(sm.Gm + r * kGS + cc);
    }
    __syncthreads();
    if constexpr (kP <= 16 && (kB == 2 || kB == 4)) {
      if (lvl > kChunk) {  // the level's scans once, at its first chunk
        if (c0 == 0) build_g_scan<E, kP, kB>(G, d, S, nq, sm.lf, sm.dls, sm.cn, sm.scv, sm.sci, tid);
        if (rcols > 0)
          build_g_emit<E, kP, kB, kXS, kGS>(G, c0, rcols, a.maxhalf, sm.Xs, sm.scv, sm.sci, sm.Gm, tid);
      } else if (rcols > 0) {
        build_g_p<E, kP, kB, kXS, kGS>(G, d, c0, rcols, S, nq, a.maxhalf, sm.Xs, sm.lf, sm.dls, sm.cn, sm.Gm, tid);
      }
    } else if (rcols > 0) {
      build_g_p<E, kP, kB, kXS, kGS>(G, d, c0, rcols, S, nq, a.maxhalf, sm.Xs, sm.lf, sm.dls, sm.cn, sm.Gm, tid);
    }
    __syncthreads();
    if (a.refc) {
      // boundary-mass gradient of the reference causal mode (ref_causal_grad_kernel)
      if (tid < nq) {
        const int t = l0 + tid;
        const int64_t qh = ((int64_t)bb * a.L + t) * a.H + h;
        const float cf = a.rc_coef[qh * T + d];
        const int base = 2 * (t >> (T - d)) - c0;  // the boundary node's left child
        if (cf != 0.f && base >= 0 && base < ncols) {
          const float xl = sm.Xs[tid * kXS + base], xr = sm.Xs[tid * kXS + base + 1];
          const float pl = 1.f / (1.f + __expf(xr - xl));
          const float rho = a.rc_rho[qh * T + d];
          const float rl = ((t >> (T - 1 - d)) & 1) ? 1.f - rho : rho;
          E* gr = sm.Gm + tid * kGS + base;
          gr[0] = (E)((float)gr[0] + cf * (rl - pl));
          gr[1] = (E)((float)gr[1] + cf * (pl - rl));
        }
      }
      __syncthreads();
    }
    {
      // G^T rows of the chunk up to the reach (without the causal restriction
      // rk covers the chunk rounded up to 32 rows, the level's zero padding
      // included), eight queries per 16-byte store
      E* gt = (E*)a.gt + (((int64_t)bh * gridDim.x + blockIdx.x) * a.nsd + G.off[lam] + c0) * kQueryTile;
      for (int e = tid; e < rk * (kQueryTile / 8); e += 256) {
        const int cc = e >> 3, q0 = (e & 7) * 8;
        E v8[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v8[i] = sm.Gm[(q0 + i) * kGS + cc];
        cp8(gt + cc * kQueryTile + q0, v8);
      }
    }
    // dq^T += C^T G^T: A = C^T rows (head dims, registers), B = G rows (LDS)
#pragma unroll
    for (int ks = 0; ks < KT; ++ks) {
      if (ks < rk / M::K) {
        F bg[4];
#pragma unroll
        for (int qt = 0; qt < 4; ++qt) bg[qt] = ld_frag(sm.Gm + (16 * qt + col) * kGS + ks * M::K + M::KPL * g);
#pragma unroll
        for (int i = 0; i < NMD; ++i) {
          const int md = w + 4 * i;
          if (md < D / 16) {
#pragma unroll
            for (int qt = 0; qt < 4; ++qt) dacc[i][qt] = M::mma(at[i][ks], bg[qt], dacc[i][qt]);
          }
        }
      }
    }
    if (nd < Tb) load_at(nd, nc0);
    __syncthreads();
    d = nd;
    c0 = nc0;
  }
  // stage the tree dq as [q][d], add the leaf parts, write
  constexpr int SS = D + 4;
  float* stage = sm.Xs;  // [64][D+4] fits in [64][kXS]
#pragma unroll
  for (int i = 0; i < NMD; ++i) {
    const int md = w + 4 * i;
    if (md < D / 16) {
#pragma unroll
      for (int qt = 0; qt < 4; ++qt) *(f32x4*)(stage + (16 * qt + col) * SS + 16 * md + 4 * g) = dacc[i][qt];
    }
  }
  __syncthreads();
  const E* dqp = (const E*)a.dq_part;
  E* dq = (E*)a.dq;
  for (int e = tid; e < nq * (D / 8); e += 256) {
    const int qi = e / (D / 8), d0 = (e - qi * (D / 8)) * 8;
    const int l = l0 + qi;
    const int64_t qh = ((int64_t)bb * a.L + l) * a.H + h;
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = stage[qi * SS + d0 + i];
    if (a.dqp) sum_rows8(acc, dqp + qh * S * D + d0, D, sm.cn[qi]);
    if (a.refc && Tb < T) {
      // boundary-mass gradient at the band depths: dq += g (c_left - c_right) = 2 g c_left
      for (int dd = Tb; dd < T; ++dd) {
        const float gv = a.rc_g[qh * T + dd];
        if (gv == 0.f) continue;
        const float* cl = a.sum32 + ((int64_t)bh * rows + G.off[dd + 1] + 2 * (l >> (T - dd))) * D + d0;
        const float4 x0 = *(const float4*)cl, x1 = *(const float4*)(cl + 4);
        acc[0] += 2.f * gv * x0.x; acc[1] += 2.f * gv * x0.y; acc[2] += 2.f * gv * x0.z; acc[3] += 2.f * gv * x0.w;
        acc[4] += 2.f * gv * x1.x; acc[5] += 2.f * gv * x1.y; acc[6] += 2.f * gv * x1.z; acc[7] += 2.f * gv * x1.w;
      }
    }
    if (a.dq32) {
      acc8f(a.dq32 + qh * D + d0, acc, a.first);
      continue;
    }
    E* o = dq + bb * a.qsb + (int64_t)l * a.qsl + h * a.qsh + d0;
    if constexpr (sizeof(E) == 2) {
      typedef __attribute__((ext_vector_type(8))) E e8;
      e8 v;
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = (E)acc[i];
      *(e8*)o = v;
    } else {
      *(float4*)o = make_float4(acc[0], acc[1], acc[2], acc[3]);
      *(float4*)(o + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
    }
  }
}

// dC partial of one query split: dsum_part[split][bh][r][:] = sum over the
// split's queries of G^T[r][q] Q[q][:].  grid (row chunks, qsplit, BH), eight
// waves; a row chunk is 8 * kDcRows row tiles of 16 summary rows and wave w
// owns tiles w, w + 8, ... of it for every head dim.  Split s takes the query
// blocks s, s + qsplit, s + 2 qsplit, ..., so under causal masking (late
// blocks reach more rows) every split gets the same mix.  Per block of queries
// the Q^T block is staged once in LDS (double-buffered: the next block's
// global loads are in flight while the current one is multiplied) and every
// G^T row is read once, straight from global memory into MFMA fragments.
constexpr int kDcRows = 3;   // row tiles per wave
constexpr int kDcKB = 64;    // queries per staged block (whole 128-byte lines of G^T rows)
static_assert(kDcKB == kQueryTile, "a staged query block is one tree_dq_kernel tile (the causal row rule)");

template <typename E, int D>
__global__ __launch_bounds__(512) void tree_dc_kernel(TreeArgs a) {
  using M = Mfma<E>;
  using F = typename M::frag;
  constexpr int KS = kDcKB / M::K;           // MFMA k-steps per block
  constexpr int QS = kDcKB + 8;              // padded LDS row stride (elements)
  constexpr int NDT = D / 16;
  constexpr int NLD = D * (kDcKB / 8);       // 8-element pieces of a Q^T block
  constexpr int PER = (NLD + 511) / 512;     // pieces per thread
  __shared__ __align__(16) E qs[2][D * QS];
  const int chunk = blockIdx.x, split = blockIdx.y, bh = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, col = lane & 15, g = lane >> 4;
  const int rows = a.nsd, ntile = rows / 16;  // the dense levels' rows
  const int64_t Lp = a.Lp;
  const int64_t nblk = Lp / kDcKB, qs_ = a.qsplit;
  const int64_t nj = split < nblk ? (nblk - split + qs_ - 1) / qs_ : 0;  // this split's query blocks
  auto kb_of = [&](int64_t j) { return (j * qs_ + split) * kDcKB; };
  const int rt0 = chunk * 8 * kDcRows + w;
  const E* gt = (const E*)a.gt + (int64_t)bh * rows * Lp;  // [query block][row][kDcKB]
  // Exact causal mode: tree_dq_kernel writes the G^T row of column c of level
  // lam for a query block only where (c & ~31) is below that block's reach,
  // i.e. where ((c & ~31) >> lb) << lb (T - lam + 1) <= blk_hi, the block's
  // last reachable leaf block; other rows may hold stale data and are neither
  // read nor multiplied.  thr() is that bound per row; the loop starts at the
  // first query block any tile of this chunk needs (blk_hi grows with kb).
  const Geo& G = a.geo;
  const bool cz = a.causal;
  auto thr = [&](int lam, int r) { return (((r - G.off[lam]) & ~31) >> G.lb) << (G.lb * (G.T - lam + 1)); };
  auto level_of = [&](int r) {
    int lam = 1;
    while (lam < G.T && r >= G.off[lam + 1]) ++lam;
    return lam;
  };
  auto bhi = [&](int64_t kb) {
    const int l0 = (int)kb, nq = min(kQueryTile, a.L - l0);
    return (l0 + nq - 1 + (a.N - a.L)) / G.LB;
  };
  int th[kDcRows];
#pragma unroll
  for (int i = 0; i < kDcRows; ++i) {
    const int r = 16 * (rt0 + 8 * i);
    th[i] = cz && r < rows ? thr(level_of(r), r) : 0;
  }
  int64_t j0 = 0;
  if (cz && nj > 0) {
    const int r0 = chunk * 8 * kDcRows * 16, r1 = min(rows, r0 + 8 * kDcRows * 16);
    int mth = 0x7fffffff;
    for (int lam = 1; lam <= G.T; ++lam) {
      const int lo = max(r0, G.off[lam]), hi = min(r1, G.off[lam + 1]);
      if (lo < hi) mth = min(mth, thr(lam, lo));
    }
    int64_t lo = 0, hi = nj;  // first j in [0, nj) with bhi >= mth (nj if none)
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (bhi(kb_of(mid)) >= mth) hi = mid;
      else lo = mid + 1;
    }
    j0 = lo;
  }
  auto need = [&](int i, int bk) { return !cz || bk >= th[i]; };
  const E* qt = (const E*)a.qt + (int64_t)bh * D * Lp;    // [query block][D][kDcKB]

  f32x4 acc[kDcRows][NDT];
#pragma unroll
  for (int i = 0; i < kDcRows; ++i)
#pragma unroll
    for (int nd = 0; nd < NDT; ++nd) acc[i][nd] = zero4();

  E qreg[PER][8];
  F af[kDcRows][KS], an[kDcRows][KS];
  auto load_q = [&](int64_t kb) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int e = tid + 512 * j;
      if (e < NLD) cp8(qreg[j], qt + kb * D + e * 8);
    }
  };
  auto store_q = [&](int buf) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int e = tid + 512 * j;
      if (e < NLD) cp8(qs[buf] + (e / (kDcKB / 8)) * QS + (e % (kDcKB / 8)) * 8, qreg[j]);
    }
  };
  auto load_a = [&](int64_t kb, F (&dst)[kDcRows][KS]) {
    const int bk = cz ? bhi(kb) : 0;
#pragma unroll
    for (int i = 0; i < kDcRows; ++i) {
      const int rt = rt0 + 8 * i;
      if (rt < ntile && need(i, bk)) {
        const E* ap = gt + ((kb / kDcKB) * rows + 16 * rt + col) * kDcKB + M::KPL * g;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) dst[i][ks] = ld_frag(ap + ks * M::K);
      }
    }
  };
  if (j0 < nj) {
    load_q(kb_of(j0));
    load_a(kb_of(j0), af);
  }
  int buf = 0;
  for (int64_t j = j0; j < nj; ++j, buf ^= 1) {
    const int bk = cz ? bhi(kb_of(j)) : 0;
    store_q(buf);
    __syncthreads();
    const bool more = j + 1 < nj;
    if (more) {
      load_q(kb_of(j + 1));
      load_a(kb_of(j + 1), an);
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      F bq[NDT];
#pragma unroll
      for (int nd = 0; nd < NDT; ++nd) bq[nd] = ld_frag(qs[buf] + (16 * nd + col) * QS + ks * M::K + M::KPL * g);
#pragma unroll
      for (int i = 0; i < kDcRows; ++i)
        if (rt0 + 8 * i < ntile && need(i, bk))
#pragma unroll
          for (int nd = 0; nd < NDT; ++nd) acc[i][nd] = M::mma(af[i][ks], bq[nd], acc[i][nd]);
    }
    if (more) {
#pragma unroll
      for (int i = 0; i < kDcRows; ++i)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) af[i][ks] = an[i][ks];
    }
  }
  float* out = a.dsum_part + ((int64_t)split * a.BHn + bh) * rows * D;
#pragma unroll
  for (int i = 0; i < kDcRows; ++i) {
    const int rt = rt0 + 8 * i;
    if (rt >= ntile) continue;
#pragma unroll
    for (int nd = 0; nd < NDT; ++nd)
#pragma unroll
      for (int r = 0; r < 4; ++r) out[(int64_t)(16 * rt + 4 * g + r) * D + 16 * nd + col] = acc[i][nd][r];
  }
}

// dsum rows of the dense levels (the first nsd rows of each (batch, head)) =
// sum over query splits (in split order); rows outside any level are 0.
__global__ __launch_bounds__(256) void dsum_reduce_kernel(const float* __restrict__ part, float* __restrict__ dsum,
                                                          int64_t n, int qsplit, Geo G, int D, int nsd, int first) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n) return;
  const int64_t row = e / D, bh = row / nsd, r = row - bh * nsd;
  int lam = 1;
  while (lam < G.T && r >= G.off[lam + 1]) ++lam;
  float s = 0.f;
  if (r - G.off[lam] < G.pw[lam])
    for (int k = 0; k < qsplit; ++k) s += part[(int64_t)k * n + e];
  float* o = dsum + (bh * G.NS + r) * D + (e - row * D);
  *o = first ? s : *o + s;
}

// dk[b, t, h, :] = dk_leaf + sum over the summaries that include token t.
// The summary part depends only on t's leaf block, so one thread per (leaf
// block, run of up to kAdjTok of its tokens, 8 dims) sums it once (T summary
// rows) and writes the run's tokens: one 16-byte store each for 16-bit
// outputs (the entry points require 16-byte aligned dk and strides in
// multiples of 8); grid (ceil(NL * runs * D/8 / 256), BH).
constexpr int kAdjTok = 16;
template <typename E>
__global__ __launch_bounds__(256) void pool_adjoint_kernel(TreeArgs a, int runs) {
  const Geo& G = a.geo;
  const int D = a.D;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t rest = e / (D / 8);
  const int d0 = (int)(e - rest * (D / 8)) * 8;
  const int beta = (int)(rest / runs), run = (int)(rest - (int64_t)beta * runs);
  if (beta >= G.NL) return;
  const int bh = blockIdx.y, bb = bh / a.H, h = bh - bb * a.H;
  const float* ds = a.dsum + (int64_t)bh * G.NS * D + d0;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  auto add = [&](const float4& x, const float4& y, float s) {
    acc[0] += x.x * s; acc[1] += x.y * s; acc[2] += x.z * s; acc[3] += x.w * s;
    acc[4] += y.x * s; acc[5] += y.y * s; acc[6] += y.z * s; acc[7] += y.w * s;
  };
  if (a.mode == TA_TREE_NATURAL) {
    for (int lam = 1; lam <= G.T; ++lam) {
      const int shift = G.lb * (G.T - lam);  // leaf blocks per node = 2^shift
      const float4* v = (const float4*)(ds + (int64_t)(G.off[lam] + (beta >> shift)) * D);
      add(v[0], v[1], 1.f / (float)(2 << shift));
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
      const float4* x = (const float4*)(ds + rl * D);
      const float4* y = (const float4*)(ds + (rl + 1) * D);
      const float4 x0 = x[0], x1 = x[1], y0 = y[0], y1 = y[1];
      const float s = (beta < p ? 0.25f : -0.25f) / (float)wl;
      add(make_float4(x0.x - y0.x, x0.y - y0.y, x0.z - y0.z, x0.w - y0.w),
          make_float4(x1.x - y1.x, x1.y - y1.y, x1.z - y1.z, x1.w - y1.w), s);
    }
  }
  const float inv = 1.f / (float)G.LB;
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] *= inv;
  const int t0 = beta * G.LB + run * kAdjTok, t1 = min(t0 + kAdjTok, (beta + 1) * G.LB);
  for (int t = t0; t < t1; ++t) {
    const int64_t th = ((int64_t)bb * a.N + t) * a.H + h;
    float4 l0 = make_float4(0.f, 0.f, 0.f, 0.f), l1 = l0;
    if (a.dkl) {
      const float4* lk = (const float4*)(a.dk_leaf + th * D + d0);
      l0 = lk[0];
      l1 = lk[1];
    }
    const float r[8] = {l0.x + acc[0], l0.y + acc[1], l0.z + acc[2], l0.w + acc[3],
                        l1.x + acc[4], l1.y + acc[5], l1.z + acc[6], l1.w + acc[7]};
    E* o = (E*)a.dk + bb * a.ksb + (int64_t)t * a.ksl + h * a.ksh + d0;
    if constexpr (sizeof(E) == 2) {
      typedef __attribute__((ext_vector_type(8))) E e8;
      e8 v;
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = (E)r[i];
      *(e8*)o = v;
    } else {
      *(float4*)o = make_float4(r[0], r[1], r[2], r[3]);
      *(float4*)(o + 4) = make_float4(r[4], r[5], r[6], r[7]);
    }
  }
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

// ---------------------------------------------------------------- bands ---
// The deep levels (depths Tb .. T-1, wider than dense G tiles pay for) run in
// bands of nb depths [da, da + nb), linear in the number of sampled pairs.  A
// band's work under node s of depth da is one workgroup: the subtree's
// (query, distinct leaf block) pairs are one contiguous run of the bucket
// order (pairs sorted by leaf block are sorted by node at every depth), taken
// 32 at a time, eight threads per pair (the query's distinct leaf blocks staged
// in LDS).  At depth d of the band the query's
// slots under the pair's node n form a run, and its first slot (the run's
// representative) carries the node's entries of G:
//   G[n, j] = A_j - p_j A_n
// (A_j: dl summed over the run's slots under child j, A_n over the run, p the
// node's child probabilities from x_j = q . c_{n,j} with the float summaries,
// 0 where the logit is clamped), exactly the dense levels' rule.  Then
//   dq_pair += sum_j G[n, j] c_{n,j}  (into the pair's dq row, summed per query
//                                      by tree_dq_kernel's epilogue),
//   dC_sub  += G_tile^T Q_tile        (MFMA over the tile's 64 pairs),
// and the subtree's R band rows of dC are written once at the end: one writer
// per entry and a fixed summation order, no atomics.
struct BandArgs {
  Geo geo;
  int L, H, S, da, nb, R, pair_rows, rmw;
  float maxhalf;
  const void* q;
  int64_t qsb, qsl, qsh;
  const float* sum32;
  const int* slot_leaf;
  const int* slot_count;
  const float* dl;
  const int* order;
  const int* block_start;
  void* dq_part;
  float* dsum;
  int first;  // 0: add to the summary-gradient rows (a later chunk of a problem with many samples)
};

constexpr int kBandRows = 64;  // dC rows of one band's subtree (b = 2: 5 depths, b = 4: 2)

template <typename E, int D, int kB>
__global__ __launch_bounds__(256, 2) void tree_band_kernel(BandArgs a) {
  using M = Mfma<E>;
  using F = typename M::frag;
  constexpr int TPP = 8;           // threads per pair
  constexpr int PC = 256 / TPP;    // pairs per chunk (the MFMA k of the dC product)
  constexpr int DQ = D / TPP;      // head dims per thread: 4, 8, 12 or 16
  constexpr int lb = kB == 2 ? 1 : 2;
  constexpr int GS = PC + (sizeof(E) == 2 ? 8 : 4);  // G tile row stride (elements)
  constexpr int QS = D + (sizeof(E) == 2 ? 8 : 4);   // Q tile row stride
  constexpr int NCT = D / 16;
  constexpr int NT = (kBandRows / 16) * NCT;  // output tiles at most
  constexpr int TPW = (NT + 3) / 4;
  __shared__ __align__(16) E Gt[kBandRows * GS];  // [band row][pair]
  __shared__ __align__(16) E Qs[PC * QS];         // [pair][dim]
  __shared__ int Sl[PC * kMaxSamples];            // each pair's query: its distinct leaf blocks
  __shared__ float Sd[PC * kMaxSamples];          //   and their dl
  const Geo& G = a.geo;
  const int s0 = blockIdx.x, bh = blockIdx.y, bb = bh / a.H, h = bh - bb * a.H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, col = lane & 15, g = lane >> 4;
  const int tp = tid / TPP, tq = tid % TPP;
  const int T = G.T, S = a.S, da = a.da, nb = a.nb, R = a.R;
  const int RP = (R + 15) & ~15, ntu = (RP / 16) * NCT;
  const int span = 1 << (lb * (T - da));  // leaf blocks under the subtree
  const int* bs = a.block_start + (int64_t)bh * (G.NL + 1);
  const int e_begin = bs[s0 * span], e_end = bs[(s0 + 1) * span];
  const int* ord = a.order + (int64_t)bh * a.L * S;
  const float* sum = a.sum32 + (int64_t)bh * G.NS * D;
  int* sl = Sl + tp * kMaxSamples;
  float* sd = Sd + tp * kMaxSamples;

  f32x4 acc[TPW];
#pragma unroll
  for (int k = 0; k < TPW; ++k) acc[k] = zero4();
  for (int e0 = e_begin; e0 < e_end; e0 += PC) {
    for (int e = tid; e < RP * PC; e += 256) Gt[(e / PC) * GS + (e % PC)] = (E)0.f;
    const int e = e0 + tp;
    const bool valid = e < e_end;
    const int ent = valid ? ord[e] : 0;
    const int l = ent / S, u = ent - l * S;
    const int64_t qh = ((int64_t)bb * a.L + l) * a.H + h;
    const int cnt = valid ? a.slot_count[qh] : 0;
    for (int v = tq; v < cnt; v += TPP) {
      sl[v] = a.slot_leaf[qh * S + v];
      sd[v] = a.dl[qh * S + v];
    }
    float qv[DQ];
    const E* qr = (const E*)a.q + bb * a.qsb + (int64_t)l * a.qsl + h * a.qsh + tq * DQ;
#pragma unroll
    for (int i = 0; i < DQ; i += 4) {
      if constexpr (sizeof(E) == 2) {
        typedef __attribute__((ext_vector_type(4))) E e4;
        const e4 x = valid ? *(const e4*)(qr + i) : e4{(E)0.f, (E)0.f, (E)0.f, (E)0.f};
#pragma unroll
        for (int t = 0; t < 4; ++t) qv[i + t] = (float)x[t];
        *(e4*)(Qs + tp * QS + tq * DQ + i) = x;
      } else {
        const float4 x = valid ? *(const float4*)(qr + i) : make_float4(0.f, 0.f, 0.f, 0.f);
        qv[i] = x.x; qv[i + 1] = x.y; qv[i + 2] = x.z; qv[i + 3] = x.w;
        *(float4*)(Qs + tp * QS + tq * DQ + i) = x;
      }
    }
    __syncthreads();  // the pairs' slot lists
    const int leaf = valid ? sl[u] : 0;
    float dqa[DQ];
#pragma unroll
    for (int i = 0; i < DQ; ++i) dqa[i] = 0.f;
    int rb = 0, pj = kB;  // local row base of band depth j, b^(j+1)
    for (int j = 0; j < nb; ++j, rb += pj, pj *= kB) {
      const int d = da + j, sh = lb * (T - d);
      const int n = leaf >> sh;
      const bool rep = valid && (u == 0 || (sl[u - 1] >> sh) != n);
      // the node's child logits (every lane takes part in the reductions)
      const float* cr = sum + ((int64_t)G.off[d + 1] + kB * n) * D + tq * DQ;
      float x[kB];
#pragma unroll
      for (int c = 0; c < kB; ++c) {
        if (c > 0 && a.pair_rows) {
          x[c] = -x[0];
          continue;
        }
        float p = 0.f;
#pragma unroll
        for (int i = 0; i < DQ; i += 4) {
          const float4 cv = *(const float4*)(cr + (int64_t)c * D + i);
          p += qv[i] * cv.x + qv[i + 1] * cv.y + qv[i + 2] * cv.z + qv[i + 3] * cv.w;
        }
        p += row_xor<1>(p, lane & 15);  // the pair's eight lanes
        p += row_xor<2>(p, lane & 15);
        p += row_xor<4>(p, lane & 15);
        x[c] = p;
      }
      if (!rep) continue;
      float An = 0.f, Ac[kB];
#pragma unroll
      for (int c = 0; c < kB; ++c) Ac[c] = 0.f;
      for (int v2 = u; v2 < cnt; ++v2) {
        const int lf2 = sl[v2];
        if ((lf2 >> sh) != n) break;
        const float dv = sd[v2];
        const int dig = (lf2 >> (sh - lb)) & (kB - 1);
        An += dv;
#pragma unroll
        for (int c = 0; c < kB; ++c)
          if (c == dig) Ac[c] += dv;
      }
      float mx = -__builtin_inff();
#pragma unroll
      for (int c = 0; c < kB; ++c) mx = fmaxf(mx, clamp_h(x[c], a.maxhalf));
      float ex[kB], se = 0.f;
#pragma unroll
      for (int c = 0; c < kB; ++c) {
        ex[c] = __expf(clamp_h(x[c], a.maxhalf) - mx);
        se += ex[c];
      }
      float gc[kB];
#pragma unroll
      for (int c = 0; c < kB; ++c) {
        const bool live = x[c] >= -a.maxhalf && x[c] <= a.maxhalf;
        gc[c] = live ? Ac[c] - ex[c] / se * An : 0.f;
      }
      if (a.pair_rows) {
        const float gd = gc[0] - gc[1];  // c_right = -c_left
#pragma unroll
        for (int i = 0; i < DQ; i += 4) {
          const float4 cv = *(const float4*)(cr + i);
          dqa[i] += gd * cv.x; dqa[i + 1] += gd * cv.y; dqa[i + 2] += gd * cv.z; dqa[i + 3] += gd * cv.w;
        }
      } else {
#pragma unroll
        for (int c = 0; c < kB; ++c)
#pragma unroll
          for (int i = 0; i < DQ; i += 4) {
            const float4 cv = *(const float4*)(cr + (int64_t)c * D + i);
            dqa[i] += gc[c] * cv.x; dqa[i + 1] += gc[c] * cv.y; dqa[i + 2] += gc[c] * cv.z; dqa[i + 3] += gc[c] * cv.w;
          }
      }
      if (tq == 0) {
        const int r0 = rb + kB * (n - (s0 << (lb * j)));
#pragma unroll
        for (int c = 0; c < kB; ++c) Gt[(r0 + c) * GS + tp] = (E)gc[c];
      }
    }
    if (valid) {
      E* dr = (E*)a.dq_part + (qh * S + u) * D + tq * DQ;
#pragma unroll
      for (int i = 0; i < DQ; i += 4) {
        float o[4] = {dqa[i], dqa[i + 1], dqa[i + 2], dqa[i + 3]};
        if constexpr (sizeof(E) == 2) {
          typedef __attribute__((ext_vector_type(4))) E e4;
          if (a.rmw) {
            const e4 y = *(const e4*)(dr + i);
#pragma unroll
            for (int t = 0; t < 4; ++t) o[t] += (float)y[t];
          }
          e4 v;
#pragma unroll
          for (int t = 0; t < 4; ++t) v[t] = (E)o[t];
          *(e4*)(dr + i) = v;
        } else {
          if (a.rmw) {
            const float4 y = *(const float4*)(dr + i);
            o[0] += y.x; o[1] += y.y; o[2] += y.z; o[3] += y.w;
          }
          *(float4*)(dr + i) = make_float4(o[0], o[1], o[2], o[3]);
        }
      }
    }
    __syncthreads();  // the G tile
    // dC_sub (band rows x D) += G_tile (rows x PC pairs) Q_tile (PC pairs x D)
#pragma unroll
    for (int k = 0; k < TPW; ++k) {
      const int t = w + 4 * k;
      if (t >= ntu) continue;
      const int rt = t / NCT, ct = t - rt * NCT;
#pragma unroll
      for (int ks = 0; ks < PC / M::K; ++ks) {
        const F af = ld_frag(Gt + (16 * rt + col) * GS + ks * M::K + M::KPL * g);
        F bf;
        if constexpr (M::KPL == 1) bf = Qs[(ks * M::K + g) * QS + 16 * ct + col];
        else bf = tr_frag<E>(Qs, QS, ks * M::K + 8 * g, ks * M::K + 8 * g + 4, 16 * ct, lane);
        acc[k] = M::mma(af, bf, acc[k]);
      }
    }
    __syncthreads();  // G tile, Q tile and slot lists are rewritten next chunk
  }
  // the subtree's band rows of dC: local row rb_j + r -> level da + j + 1, row s0 b^(j+1) + r
#pragma unroll
  for (int k = 0; k < TPW; ++k) {
    const int t = w + 4 * k;
    if (t >= ntu) continue;
    const int rt = t / NCT, ct = t - rt * NCT;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int lr = 16 * rt + 4 * g + r;
      if (lr >= R) continue;
      int j = 0, pj = kB;
      while (lr >= pj) {
        lr -= pj;
        pj *= kB;
        ++j;
      }
      const int64_t grow = G.off[da + j + 1] + ((int64_t)s0 << (lb * (j + 1))) + lr;
      float* o = a.dsum + ((int64_t)bh * G.NS + grow) * D + 16 * ct + col;
      *o = a.first ? acc[k][r] : *o + acc[k][r];
    }
  }
}

// Reference causal mode at the band depths: the boundary children's part of
// dC, dC[left child of n] += sum_t g_t q_t and dC[right child] -= the same,
// over the queries t whose boundary node at depth d is n (t >> (T - d) = n, a
// contiguous range; rc_g from ref_causal_grad_kernel).  One thread per (node,
// eight head dims), queries in order; runs after the band kernels wrote these
// rows.  grid (ceil(2^d D / 8 / 256), B*H).
template <typename E>
__global__ __launch_bounds__(256) void ref_band_boundary_kernel(TreeArgs a, int d) {
  const Geo& G = a.geo;
  const int D = a.D, T = G.T;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= ((int64_t)1 << d) * (D / 8)) return;
  const int bh = blockIdx.y, bb = bh / a.H, h = bh - bb * a.H;
  const int n = (int)(e / (D / 8)), d0 = (int)(e - (int64_t)n * (D / 8)) * 8;
  const int t_lo = max(n << (T - d), a.t0), t_hi = min((n + 1) << (T - d), a.L);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  bool any = false;
  for (int t = t_lo; t < t_hi; ++t) {
    const float gv = a.rc_g[(((int64_t)bb * a.L + t) * a.H + h) * T + d];
    if (gv == 0.f) continue;
    any = true;
    float qv[8];
    ld8f(qv, (const E*)a.q + bb * a.qsb + (int64_t)t * a.qsl + h * a.qsh + d0);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] += gv * qv[i];
  }
  if (!any) return;
  float* left = a.dsum + ((int64_t)bh * G.NS + G.off[d + 1] + 2 * n) * D + d0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    left[i] += acc[i];
    left[D + i] -= acc[i];
  }
}

// Path-row backward (the leaf backward added each pair's tree gradient to
// its dq row and wrote each leaf block's gradient of its path's child
// summaries, leaf_bwd_tr.h): dq[q] = the sum of the query's pair rows, in
// slot order, one thread per (query, eight head dims); written to dq (E,
// strided) or, for a chunk of a problem with many samples, to dq32.
template <typename E>
__global__ __launch_bounds__(256) void dq_rows_kernel(TreeArgs a, int64_t n8) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n8) return;
  const int D = a.D;
  const int64_t qh = e / (D / 8);
  const int d0 = (int)(e - qh * (D / 8)) * 8;
  const int64_t h = qh % a.H, bl = qh / a.H, l = bl % a.L, bb = bl / a.L;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  sum_rows8(acc, (const E*)a.dq_part + qh * a.S * D + d0, D, a.slot_count[qh]);
  if (a.dq32) {
    acc8f(a.dq32 + qh * D + d0, acc, a.first);
    return;
  }
  E* o = (E*)a.dq + bb * a.qsb + l * a.qsl + h * a.qsh + d0;
  if constexpr (sizeof(E) == 2) {
    typedef __attribute__((ext_vector_type(8))) E e8;
    e8 v;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (E)acc[i];
    *(e8*)o = v;
  } else {
    *(float4*)o = make_float4(acc[0], acc[1], acc[2], acc[3]);
    *(float4*)(o + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
}

// Path-row backward: dsum[row] for child j of the depth-d node n = the sum
// over the leaf blocks u under n (u in [n b^(T-d), (n+1) b^(T-d)), in order of
// lane) of dcp[u][d b + j]; rows padding a level are 0.  One wavefront per
// (batch * head, summary row): lanes = DG groups of eight head dims x 64 / DG
// block lanes (block lane i takes blocks lo + i, lo + i + 64 / DG, ...), then a
// butterfly over the block lanes (a fixed order: deterministic).  dcp rows
// are (BH, NL, T b, D) floats.  first = 0 (later chunks of a problem with many
// samples) adds to dsum.
// (Also the one-token leaves' per-subtree root-path rows, leaf_path1.hip: G
// then describes the tree above the subtrees -- T = depths above them, NL =
// subtrees, NS = the rows of those levels -- nr = rows per subtree and ns the
// summary-gradient rows per (batch, head).)
template <int DG>
__global__ __launch_bounds__(256) void path_dsum_kernel(const float* __restrict__ dcp, float* __restrict__ dsum,
                                                        Geo G, int D, int64_t nrows, int first, int nr, int ns) {
  const int64_t wv = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  if (wv >= nrows) return;
  const int lane = threadIdx.x & 63;
  const int64_t bh = wv / G.NS;
  const int row = (int)(wv - bh * G.NS);
  int lam = 1;
  while (lam < G.T && row >= G.off[lam + 1]) ++lam;
  const int i = row - G.off[lam];
  const int dg = lane % DG, bl = lane / DG;
  constexpr int NBL = 64 / DG;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (i < G.pw[lam] && 8 * dg < D) {
    const int d = lam - 1, j = i & (G.b - 1), n = i >> G.lb;
    const int span = G.pw[G.T - d];
    const int lo = n * span, hi = min(lo + span, G.NL);
    const float* src = dcp + ((int64_t)bh * G.NL * nr + (int64_t)d * G.b + j) * D + 8 * dg;
    for (int u = lo + bl; u < hi; u += NBL) {
      const float* x = src + (int64_t)u * nr * D;
      const float4 p0 = *(const float4*)x, p1 = *(const float4*)(x + 4);
      acc[0] += p0.x; acc[1] += p0.y; acc[2] += p0.z; acc[3] += p0.w;
      acc[4] += p1.x; acc[5] += p1.y; acc[6] += p1.z; acc[7] += p1.w;
    }
  }
#pragma unroll
  for (int o = DG; o < 64; o <<= 1)
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] += __shfl_xor(acc[k], o, 64);
  if (bl == 0 && 8 * dg < D) acc8f(dsum + ((int64_t)bh * ns + row) * D + 8 * dg, acc, first);
}

static int tree_smem(const Plan& P) {
  const int S = (int)P.S;
  // + the hoisted scan lanes (S <= 16): two floats and three ints each
  const int ch = chunk_cols((int)P.D);
  return kQueryTile * (ch + 4) * 4 + kQueryTile * (ch + 8) * P.esize + kQueryTile * S * 8 + kQueryTile * 4 +
         (S <= 8 ? kQueryTile * 8 * 20 : S <= 16 ? kQueryTile * 16 * 20 : 0);
}

static void launch_path_dsum(const float* dcp, float* dsum, const Geo& G, int D, int64_t BH, int first, int nr,
                             int ns, hipStream_t st) {
  const int64_t nrows = BH * G.NS;
  const dim3 grid((unsigned)((nrows + 3) / 4));
  if (D <= 32) hipLaunchKernelGGL(path_dsum_kernel<4>, grid, dim3(256), 0, st, dcp, dsum, G, D, nrows, first, nr, ns);
  else if (D <= 64) hipLaunchKernelGGL(path_dsum_kernel<8>, grid, dim3(256), 0, st, dcp, dsum, G, D, nrows, first, nr, ns);
  else hipLaunchKernelGGL(path_dsum_kernel<16>, grid, dim3(256), 0, st, dcp, dsum, G, D, nrows, first, nr, ns);
}

// dk from the summary gradient (and the leaf part): once per problem, after
// the last chunk of a problem with many samples.
template <typename E>
static hipError_t tree_adjoint(const Plan& P, const TreeArgs& a, bool chunk, hipStream_t st) {
  if (chunk && !P.acc.last) return hipGetLastError();
  const int D = a.D;
  if (P.p.tree_mode == TA_TREE_NODEKEYS) {
    const int64_t n = (int64_t)(P.geo.NL - 1) * D;
    if (n > 0)
      hipLaunchKernelGGL(nodekeys_adjoint_kernel<E>, dim3((unsigned)((n + 255) / 256), P.BH), dim3(256), 0, st, a);
  } else {
    const int runs = (P.geo.LB + kAdjTok - 1) / kAdjTok;
    const int64_t n = (int64_t)P.geo.NL * runs * (D / 8);
    hipLaunchKernelGGL(pool_adjoint_kernel<E>, dim3((unsigned)((n + 255) / 256), P.BH), dim3(256), 0, st, a, runs);
  }
  return hipGetLastError();
}

template <typename E, int D>
static hipError_t tree_impl(const Plan& P, const void* q, const char* rec, void* dq, void* dk, char* ws,
                            hipStream_t st) {
  TreeArgs a;
  a.geo = P.geo;
  a.L = (int)P.L;
  a.N = (int)P.N;
  a.H = (int)P.H;
  a.S = (int)P.S;
  a.D = D;
  a.causal = P.p.causal == TA_CAUSAL_EXACT;
  a.mode = P.p.tree_mode;
  a.maxhalf = 0.5f * P.p.max_logit;
  a.q = q;
  a.qsb = P.p.q_strides[0]; a.qsl = P.p.q_strides[1]; a.qsh = P.p.q_strides[2];
  a.sum_hi = sizeof(E) == 2 ? (const void*)(rec + P.rec.sum_hi) : (const void*)(rec + P.rec.summaries);
  a.sum_t = rec + P.rec.sum_t;
  a.slot_leaf = (const int*)(rec + P.rec.slot_leaf);
  a.slot_count = (const int*)(rec + P.rec.slot_count);
  a.slot_weight = (const float*)(rec + P.rec.slot_weight);
  a.delta = (const float*)(ws + P.bws.delta);
  a.dq_part = ws + P.bws.dq_part;
  a.dl = (float*)(ws + P.bws.dlogp);
  a.gt = ws + P.bws.gt;
  a.qt = ws + P.bws.qt;
  a.Lp = P.Lp;
  a.dq = dq;
  a.dsum_part = (float*)(ws + P.bws.dsum_part);
  const bool chunk = P.acc.dq32 != nullptr;  // a chunk of a problem with many samples
  a.dsum = chunk ? P.acc.dsum : (float*)(ws + P.bws.dsum);
  a.dk_leaf = chunk ? P.acc.dk_leaf : (const float*)(ws + P.bws.dk_leaf);
  a.dq32 = P.acc.dq32;
  a.first = chunk ? P.acc.first : 1;
  a.dk = dk;
  a.ksb = P.p.k_strides[0]; a.ksl = P.p.k_strides[1]; a.ksh = P.p.k_strides[2];
  a.qsplit = P.qsplit;
  a.BHn = (int)P.BH;
  a.refc = P.p.causal == TA_CAUSAL_REFERENCE;
  a.t0 = P.L > P.S ? (int)P.S : 0;
  a.nqh = P.B * P.L * P.H;
  a.sum32 = (const float*)(rec + P.rec.summaries);
  a.dstar = (const int*)(rec + P.rec.dstar);
  a.rc_coef = (float*)(ws + P.bws.rc_coef);
  a.rc_rho = (float*)(ws + P.bws.rc_rho);
  a.rc_g = (float*)(ws + P.bws.rc_g);
  a.Tb = P.tree_dense;
  a.nsd = P.geo.off[P.tree_dense + 1];
  a.dqp = P.geo.LB > 1 || P.tree_dense < P.geo.T;
  a.dkl = P.geo.LB > 1 && P.p.tree_mode != TA_TREE_NODEKEYS;

  const int64_t nqh = P.B * P.L * P.H;
  if (P.path_rows) {
    // the leaf backward added the tree gradient: sum the pairs' dq rows and
    // the leaf blocks' path rows under each node, then the key adjoint
    a.dcp = (const float*)(ws + P.bws.dcp);
    const int64_t n8 = nqh * (D / 8);
    hipLaunchKernelGGL(dq_rows_kernel<E>, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, st, a, n8);
    launch_path_dsum(a.dcp, a.dsum, P.geo, D, P.BH, a.first, P.geo.T * P.geo.b, P.geo.NS, st);
    return tree_adjoint<E>(P, a, chunk, st);
  }
  int pw2 = 1;
  while (pw2 < P.S) pw2 <<= 1;
  hipLaunchKernelGGL(slot_dlogp_kernel, dim3((unsigned)((nqh * pw2 + 255) / 256)), dim3(256), 0, st, a.slot_count,
                     a.slot_weight, a.delta, a.dl, (int)P.S, pw2, nqh, P.acc.mean);
  if (P.leaf_path) {
    // one-token leaves: the tree gradient along the paths per subtree of
    // 2^g leaves, the root-path rows summed over the subtrees under each
    // node, dq from the pairs' rows, then the key adjoint
    hipError_t e = launch_leaf_path1(P, q, rec, ws, a.dsum, a.first, st);
    if (e != hipSuccess) return e;
    const int g = P.leaf_path;
    if (P.geo.T > g) {
      Geo top = P.geo;
      top.T = P.geo.T - g;
      top.NL = P.geo.NL >> g;
      top.NS = P.geo.off[top.T + 1];
      launch_path_dsum((const float*)(ws + P.bws.dcp), a.dsum, top, D, P.BH, a.first, leaf_path1_top_rows(), P.geo.NS,
                       st);
    }
    const int64_t n8 = nqh * (D / 8);
    hipLaunchKernelGGL(dq_rows_kernel<E>, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, st, a, n8);
    return tree_adjoint<E>(P, a, chunk, st);
  }
  if (a.refc)
    hipLaunchKernelGGL(ref_causal_grad_kernel<E>, dim3((unsigned)((nqh + 255) / 256)), dim3(256), 0, st, a);
  // the band depths (before tree_dq_kernel, whose epilogue sums the pairs' dq rows)
  if (P.tree_dense < P.geo.T) {
    const int b = P.geo.b, nbmax = b == 2 ? 5 : 2;
    BandArgs ba;
    ba.geo = P.geo;
    ba.L = (int)P.L;
    ba.H = (int)P.H;
    ba.S = (int)P.S;
    ba.pair_rows = P.p.tree_mode != TA_TREE_NATURAL && b == 2;
    ba.maxhalf = a.maxhalf;
    ba.q = q;
    ba.qsb = a.qsb; ba.qsl = a.qsl; ba.qsh = a.qsh;
    ba.sum32 = (const float*)(rec + P.rec.summaries);
    ba.slot_leaf = a.slot_leaf;
    ba.slot_count = a.slot_count;
    ba.dl = a.dl;
    ba.order = (const int*)(rec + P.rec.order);
    ba.block_start = (const int*)(rec + P.rec.block_start);
    ba.dq_part = ws + P.bws.dq_part;
    ba.dsum = a.dsum;
    ba.first = a.first;
    for (int da = P.tree_dense; da < P.geo.T; da += nbmax) {
      ba.da = da;
      ba.nb = P.geo.T - da < nbmax ? P.geo.T - da : nbmax;
      ba.R = 0;
      for (int j = 0, pj = b; j < ba.nb; ++j, pj *= b) ba.R += pj;
      ba.rmw = P.geo.LB > 1 || da > P.tree_dense;  // leaf dq rows exist, or an earlier band wrote them
      const dim3 grid((unsigned)P.geo.pw[da], (unsigned)P.BH);
      if (b == 2) hipLaunchKernelGGL((tree_band_kernel<E, D, 2>), grid, dim3(256), 0, st, ba);
      else hipLaunchKernelGGL((tree_band_kernel<E, D, 4>), grid, dim3(256), 0, st, ba);
    }
  }
  const int smem_q = tree_smem(P);
  const unsigned qtiles = (unsigned)(P.Lp / kQueryTile);
  auto launch_dq = [&](auto kern) -> hipError_t {
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, smem_q);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3(qtiles, P.BH), dim3(256), smem_q, st, a);
    return hipSuccess;
  };
  hipError_t e = hipSuccess;
  if (P.S > 32 && P.geo.b == 2) e = launch_dq(tree_dq_kernel<E, D, 64, 2>);
  else if (P.S > 32 && P.geo.b == 4) e = launch_dq(tree_dq_kernel<E, D, 64, 4>);
  else if (P.S > 32) e = launch_dq(tree_dq_kernel<E, D, 64, 0>);
  else if (P.S > 16 && P.geo.b == 2) e = launch_dq(tree_dq_kernel<E, D, 32, 2>);
  else if (P.S > 16 && P.geo.b == 4) e = launch_dq(tree_dq_kernel<E, D, 32, 4>);
  else if (P.S > 16) e = launch_dq(tree_dq_kernel<E, D, 32, 0>);
  else if (P.S <= 8 && P.geo.b == 2) e = launch_dq(tree_dq_kernel<E, D, 8, 2>);  // half the scan lanes
  else if (P.S <= 8 && P.geo.b == 4) e = launch_dq(tree_dq_kernel<E, D, 8, 4>);
  else if (P.geo.b == 4) e = launch_dq(tree_dq_kernel<E, D, 16, 4>);
  else if (P.geo.b == 2) e = launch_dq(tree_dq_kernel<E, D, 16, 2>);
  else e = launch_dq(tree_dq_kernel<E, D, 16, 0>);
  if (e != hipSuccess) return e;
  if (a.refc)
    for (int d = P.tree_dense; d < P.geo.T; ++d) {
      const int64_t n = ((int64_t)1 << d) * (D / 8);
      hipLaunchKernelGGL(ref_band_boundary_kernel<E>, dim3((unsigned)((n + 255) / 256), P.BH), dim3(256), 0, st, a,
                         d);
    }
  if (a.nsd > 0) {
    const unsigned chunks = (unsigned)((a.nsd / 16 + 8 * kDcRows - 1) / (8 * kDcRows));
    hipLaunchKernelGGL((tree_dc_kernel<E, D>), dim3(chunks, P.qsplit, P.BH), dim3(512), 0, st, a);
    const int64_t n = P.BH * (int64_t)a.nsd * D;
    hipLaunchKernelGGL(dsum_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       (const float*)a.dsum_part, a.dsum, n, P.qsplit, P.geo, D, a.nsd, a.first);
  }
  return tree_adjoint<E>(P, a, chunk, st);
}

template <typename E>
static hipError_t tree_d(const Plan& P, const void* q, const char* rec, void* dq, void* dk, char* ws, hipStream_t st) {
  switch (P.D) {
    case 32: return tree_impl<E, 32>(P, q, rec, dq, dk, ws, st);
    case 64: return tree_impl<E, 64>(P, q, rec, dq, dk, ws, st);
    case 96: return tree_impl<E, 96>(P, q, rec, dq, dk, ws, st);
    default: return tree_impl<E, 128>(P, q, rec, dq, dk, ws, st);
  }
}

hipError_t launch_tree_bwd(const Plan& P, const void* q, const float* weights, const char* rec, void* dq, void* dk,
                           char* ws, hipStream_t st) {
  (void)weights;  // the record's summed weight per distinct leaf block carries what the backward needs
  switch (P.p.dtype) {
    case TA_F32: return tree_d<float>(P, q, rec, dq, dk, ws, st);
    case TA_BF16: return tree_d<bf16>(P, q, rec, dq, dk, ws, st);
    default: return tree_d<f16>(P, q, rec, dq, dk, ws, st);
  }
}

}  // namespace ta
