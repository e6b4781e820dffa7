// Tree gradient along the sampled paths for one-token leaves (leaf_block 1,
// binary: the reference's own tree), 16-bit inputs.
//
// The reference walks every sample's path in the backward
// (_autograd.py:789-856, accumulate_qk_non_causal_all_depths_prepared.cu:
// 132-161): per depth the chosen child's logit gets dl (1 - p), the other
// -dl p, dq += gamma k_node and dk_node += gamma q.  Here the pairs (query,
// distinct leaf) are grouped by leaf (the bucket order), so the pairs of 2^g
// consecutive leaves -- a subtree of depth g at the bottom of the tree -- are
// one contiguous run, and one workgroup takes them in tiles of 128:
//   * the subtree's root path (depths 0 .. T - g - 1) is the same for all of
//     its pairs: its 2 (T - g) child summaries are rows 0 .. 31 of a path
//     tile (up to 16 depths above the subtree);
//   * the subtree's own 2^(g+1) - 2 child summaries (depths T - g .. T - 1)
//     are rows 32 .. 159; a pair's path crosses 2 g of them.
// Per tile X = C Q^T (160 rows x the pairs, MFMA), per pair and depth on its
// path gamma_j = dl ([j on the path] - p_j) (0 where the logit was clamped and
// on rows off the path), dq_pair = C^T gamma (MFMA, k = rows) into the pair's
// dq row, and dC += gamma^T Q over the tile's pairs (MFMA) with the Q rows
// and gamma staged in LDS.  dl is the per-slot log-prob gradient of
// slot_dlogp_kernel.  The subtree's own rows of dC belong to this workgroup
// alone and go straight to the summary gradient; the root-path rows go to a
// per-subtree table that path_dsum_kernel sums over the subtrees under each
// node.  No atomics; every sum in a fixed order.
#include "launch.h"

namespace ta {

constexpr int kP1Top = 32;    // root-path rows (2 (T - g) used)
constexpr int kP1Bot = 128;   // subtree rows (2^(g+1) - 2 used)
constexpr int kP1Rows = kP1Top + kP1Bot;
constexpr int kP1Tiles = kP1Rows / 16;
constexpr int kP1QT = 128;    // pairs per tile, 16 per wave
constexpr int kP1G = 6;       // subtree depth (2^(kP1G+1) - 2 <= kP1Bot)
static_assert((2 << kP1G) - 2 <= kP1Bot, "subtree rows");

struct Path1Args {
  Geo geo;
  int L, H, S, g, nsub;
  float maxhalf;
  const void* q;
  int64_t qsb, qsl, qsh;
  const void* sum_hi;  // E (BH, NS, D)
  const int* order;
  const int* block_start;
  const int* slot_leaf;
  const float* dl;     // (B, L, H, S)
  void* dq_part;       // E (B, L, H, S, D)
  float* dsum;         // (BH, NS, D)
  float* dct;          // (BH, nsub, kP1Top, D)
  int first;
};

// Summary row of path-tile row e of subtree sub (-1: unused row).
__device__ __forceinline__ int p1_row(const Geo& G, int g, int sub, int e) {
  const int T = G.T;
  if (e < kP1Top) {
    const int d = e >> 1;
    if (d >= T - g) return -1;
    return G.off[d + 1] + ((sub >> (T - g - d)) << 1) + (e & 1);
  }
  const int r = e - kP1Top;
  if (r >= (2 << g) - 2) return -1;
  const int k = 31 - __clz(r + 2) - 1;  // depth T - g + k inside the subtree
  return G.off[T - g + k + 1] + (sub << (k + 1)) + (r - ((2 << k) - 2));
}

template <typename E, int D>
__global__ __launch_bounds__(512) void path1_kernel(Path1Args a) {
  using M = Mfma<E>;
  constexpr int RS = D + 16, GS = kP1Rows + 16;
  extern __shared__ __align__(16) char smem[];
  E* Cs = (E*)smem;            // [160][RS]  path rows
  E* Qs = Cs + kP1Rows * RS;   // [128][RS]  Q rows of the tile
  E* Gm = Qs + kP1QT * RS;     // [128][GS]  gamma of the tile's pairs

  const Geo& G = a.geo;
  const int sub = blockIdx.x, bh = blockIdx.y, bb = bh / a.H, h = bh - bb * a.H;
  const int T = G.T, g = a.g, S = a.S;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, col = lane & 15, gq = lane >> 4;
  const int* bs = a.block_start + (int64_t)bh * (G.NL + 1);
  const int lo = sub << g, start = bs[lo], end = bs[min(lo + (1 << g), G.NL)];

  {  // stage the path rows
    constexpr int NST = (kP1Rows * D / 8 + 511) / 512;
    uint4 cr[NST];
#pragma unroll
    for (int i = 0; i < NST; ++i) {
      const int e = tid + i * 512;
      const int row = e / (D / 8), c = (e - row * (D / 8)) * 8;
      const int sr = e < kP1Rows * D / 8 ? p1_row(G, g, sub, row) : -1;
      cr[i] = sr >= 0 ? *(const uint4*)((const E*)a.sum_hi + ((int64_t)bh * G.NS + sr) * D + c)
                      : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < NST; ++i) {
      const int e = tid + i * 512;
      const int row = e / (D / 8), c = (e - row * (D / 8)) * 8;
      if (e < kP1Rows * D / 8) *(uint4*)(Cs + row * RS + c) = cr[i];
    }
  }
  __syncthreads();

  // phase B: dC tiles (row tile, head-dim tile), wave w takes w, w + 8, ...
  constexpr int NDT = D / 16, NT = kP1Tiles * NDT, NTW = (NT + 7) / 8;
  f32x4 cacc[NTW];
#pragma unroll
  for (int i = 0; i < NTW; ++i) cacc[i] = zero4();

  const int* ord = a.order + (int64_t)bh * a.L * S;
  const int pcol = 16 * w + col;
  const E* q = (const E*)a.q;
  for (int t0 = start; t0 < end; t0 += kP1QT) {
    const int e = t0 + pcol < end ? ord[t0 + pcol] : -1;
    const int l = e >= 0 ? e / S : 0;
    const int64_t sl = (((int64_t)bb * a.L + l) * a.H + h) * S + (e >= 0 ? e - l * S : 0);
    RowFrags<E, D> qc;
    qc.load(e >= 0 ? q + bb * a.qsb + (int64_t)l * a.qsl + h * a.qsh : nullptr, gq);
    const int leaf = e >= 0 ? a.slot_leaf[sl] : lo;
    const float dl = e >= 0 ? a.dl[sl] : 0.f;
    const int loc = leaf - lo;  // the pair's leaf inside the subtree

    // ---- X = C Q^T: rows 16 t + 4 gq + r of this lane's pair column
    f32x4 x[kP1Tiles];
#pragma unroll
    for (int t = 0; t < kP1Tiles; ++t) {
      x[t] = zero4();
      const E* cp = Cs + (16 * t + col) * RS + M::KPL * gq;
#pragma unroll
      for (int ks = 0; ks < D / M::K; ++ks) x[t] = M::mma(ld_frag(cp + ks * M::K), qc.f[ks], x[t]);
    }
    // ---- gamma on the pair's path (rows in child pairs 2i, 2i + 1: lanes
    // hold rows 4 gq + 0, 1 and 4 gq + 2, 3)
#pragma unroll
    for (int t = 0; t < kP1Tiles; ++t) {
#pragma unroll
      for (int hp = 0; hp < 2; ++hp) {
        const int e0 = 16 * t + 4 * gq + 2 * hp;  // the node's left child row
        bool on = false;
        int jp = 0;
        if (e0 < kP1Top) {
          const int d = e0 >> 1;
          on = d < T - g;
          jp = on ? (leaf >> (T - 1 - d)) & 1 : 0;
        } else {
          const int r = e0 - kP1Top;
          if (r < (2 << g) - 2) {
            const int k = 31 - __clz(r + 2) - 1;
            const int i = (r - ((2 << k) - 2)) >> 1;  // node at depth T - g + k, inside the subtree
            on = i == (loc >> (g - k));
            jp = (loc >> (g - k - 1)) & 1;
          }
        }
        const float x0 = x[t][2 * hp], x1 = x[t][2 * hp + 1];
        float g0 = 0.f, g1 = 0.f;
        if (on) {
          const float c0 = fminf(fmaxf(x0, -a.maxhalf), a.maxhalf), c1 = fminf(fmaxf(x1, -a.maxhalf), a.maxhalf);
          const float mx = fmaxf(c0, c1);
          const float e0v = __expf(c0 - mx), e1v = __expf(c1 - mx);
          const float pa = dl / (e0v + e1v);
          const bool l0 = x0 >= -a.maxhalf && x0 <= a.maxhalf, l1 = x1 >= -a.maxhalf && x1 <= a.maxhalf;
          g0 = l0 ? (jp == 0 ? dl : 0.f) - e0v * pa : 0.f;
          g1 = l1 ? (jp == 1 ? dl : 0.f) - e1v * pa : 0.f;
        }
        x[t][2 * hp] = g0;
        x[t][2 * hp + 1] = g1;
      }
    }
    // ---- dq_pair^T = C^T gamma^T (k = rows; each lane ends with eight
    // consecutive dims of its pair's row)
    E* dqp = (E*)a.dq_part + sl * D + 8 * gq;
#pragma unroll
    for (int p = 0; p < D / 32; ++p) {
      f32x4 o0 = zero4(), o1 = zero4();
#pragma unroll
      for (int ks = 0; ks < kP1Rows / M::K; ++ks) {
        const typename M::frag z = acc_operand<E>(x, ks);
        o0 = M::mma(perm_dim_frag<E>(Cs, RS, 2 * p, ks, lane), z, o0);
        o1 = M::mma(perm_dim_frag<E>(Cs, RS, 2 * p + 1, ks, lane), z, o1);
      }
      if (e >= 0) {
        typedef __attribute__((ext_vector_type(8))) E e8;
        e8 o;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          o[r] = (E)o0[r];
          o[4 + r] = (E)o1[r];
        }
        *(e8*)(dqp + 32 * p) = o;
      }
    }
    __syncthreads();  // phase B of the previous tile is done with Qs / Gm
#pragma unroll
    for (int ks = 0; ks < D / M::K; ++ks)
      *(typename M::frag*)(Qs + pcol * RS + ks * M::K + M::KPL * gq) = qc.f[ks];
#pragma unroll
    for (int t = 0; t < kP1Tiles; ++t) {
      typedef __attribute__((ext_vector_type(4))) E e4;
      e4 v;
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = (E)x[t][r];
      *(e4*)(Gm + pcol * GS + 16 * t + 4 * gq) = v;
    }
    __syncthreads();
    // ---- phase B: dC += gamma^T Q over the tile's pairs
#pragma unroll
    for (int ks = 0; ks < kP1QT / M::K; ++ks) {
      const int ka = 32 * ks + 8 * gq, kb = ka + 4;
#pragma unroll
      for (int i = 0; i < NTW; ++i) {
        const int tt = w + 8 * i;
        if (NT % 8 == 0 || tt < NT) {
          const int rt = tt / NDT, dt = tt - rt * NDT;
          cacc[i] = M::mma(tr_frag(Gm, GS, ka, kb, 16 * rt, lane), tr_frag(Qs, RS, ka, kb, 16 * dt, lane), cacc[i]);
        }
      }
    }
  }

  // root-path rows to the per-subtree table, subtree rows to the summary gradient
#pragma unroll
  for (int i = 0; i < NTW; ++i) {
    const int tt = w + 8 * i;
    if (NT % 8 == 0 || tt < NT) {
      const int rt = tt / NDT, dt = tt - rt * NDT;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int e = 16 * rt + 4 * gq + r, d = 16 * dt + col;
        if (e < kP1Top) {
          a.dct[(((int64_t)bh * a.nsub + sub) * kP1Top + e) * D + d] = cacc[i][r];
        } else {
          const int sr = p1_row(G, g, sub, e);
          if (sr >= 0) {
            float* o = a.dsum + ((int64_t)bh * G.NS + sr) * D + d;
            *o = a.first ? cacc[i][r] : *o + cacc[i][r];
          }
        }
      }
    }
  }
}

static int path1_smem(int D) { return (kP1Rows * (D + 16) + kP1QT * (D + 16) + kP1QT * (kP1Rows + 16)) * 2; }

int leaf_path1_depth(int T) { return T < kP1G ? T : kP1G; }
int leaf_path1_top_rows() { return kP1Top; }
int leaf_path1_smem(int D) { return path1_smem(D); }

template <typename E, int D>
static hipError_t path1_t(const Plan& P, const void* q, const char* rec, char* ws, float* dsum, int first,
                          hipStream_t st) {
  Path1Args a;
  a.geo = P.geo;
  a.L = (int)P.L;
  a.H = (int)P.H;
  a.S = (int)P.S;
  a.g = P.leaf_path;
  a.nsub = P.geo.NL >> P.leaf_path;
  a.maxhalf = 0.5f * P.p.max_logit;
  a.q = q;
  a.qsb = P.p.q_strides[0]; a.qsl = P.p.q_strides[1]; a.qsh = P.p.q_strides[2];
  a.sum_hi = rec + P.rec.sum_hi;
  a.order = (const int*)(rec + P.rec.order);
  a.block_start = (const int*)(rec + P.rec.block_start);
  a.slot_leaf = (const int*)(rec + P.rec.slot_leaf);
  a.dl = (const float*)(ws + P.bws.dlogp);
  a.dq_part = ws + P.bws.dq_part;
  a.dsum = dsum;
  a.dct = (float*)(ws + P.bws.dcp);
  a.first = first;
  const int smem = path1_smem(D);
  hipError_t e = hipFuncSetAttribute((const void*)path1_kernel<E, D>, hipFuncAttributeMaxDynamicSharedMemorySize, smem);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((path1_kernel<E, D>), dim3((unsigned)a.nsub, (unsigned)P.BH), dim3(512), smem, st, a);
  return hipGetLastError();
}

template <typename E>
static hipError_t path1_d(const Plan& P, const void* q, const char* rec, char* ws, float* dsum, int first,
                          hipStream_t st) {
  switch (P.D) {
    case 32: return path1_t<E, 32>(P, q, rec, ws, dsum, first, st);
    case 64: return path1_t<E, 64>(P, q, rec, ws, dsum, first, st);
    case 96: return path1_t<E, 96>(P, q, rec, ws, dsum, first, st);
    default: return path1_t<E, 128>(P, q, rec, ws, dsum, first, st);
  }
}

hipError_t launch_leaf_path1(const Plan& P, const void* q, const char* rec, char* ws, float* dsum, int first,
                             hipStream_t st) {
  switch (P.p.dtype) {
    case TA_BF16: return path1_d<bf16>(P, q, rec, ws, dsum, first, st);
    case TA_F16: return path1_d<f16>(P, q, rec, ws, dsum, first, st);
    default: return hipErrorInvalidValue;  // 16-bit inputs only (make_plan)
  }
}

}  // namespace ta
