// K2: per-query root-to-leaf path sampling (kernel templates, shared by
// sample.hip and sample_replay.hip so the two variants compile in parallel).
//
// Generalizes _sample_paths_non_causal (_tree_mha.py:78-122) and the
// treeattn-cuda step kernel (sample_non_causal_paths.cu:54-128) to b-ary trees
// with leaf blocks.  One workgroup owns 64 consecutive queries of one
// (batch, head); every thread owns a fixed set of (query, sample) items whose
// current node and accumulated log-probability stay in registers for the
// whole walk.  Per depth:
//   1. the child logits of every node of the level that the tile can reach
//      are one MFMA product  C_level (rows) x Q^T (64 queries), each wave
//      taking every fourth 16-row tile of C for all 64 queries, so every
//      summary row is read once per workgroup.  Summaries are split into
//      hi + lo parts of the input type so the logits are float-accurate.
//      The tile lands in LDS as X[query][child].
//   2. each item reads its node's b child logits from LDS and decides:
//        logp_j = log_softmax(clamp(x_j, +-max_logit/2))  (+ the causal
//        correction on the boundary path),
//        direction = argmax_j(logp_j + g_j), first maximum wins,
//      with g = -log(-log u) from the caller's uniforms or the counter RNG.
// Finally each item computes its sample weight (softmax over the query's
// samples, _tree_mha.py:396-399) and the query's ascending distinct leaf
// blocks with their summed weights, through LDS.
#pragma once

#include "launch.h"

namespace ta {

struct SampleArgs {
  Geo geo;
  int B, L, H, S, causal, coff;  // coff = N - L: causal offset of query positions
  int s0, stot;   // this launch's samples are s0 .. s0 + S - 1 of stot (uniform and path indexing)
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
  float* lse;            // (B, L, H): log of the sum over the query's samples of exp(log-prob)
  const uint8_t* paths;  // replay: packed path bits (L, B, H, S, nbytes), else null
  int nbits, nbytes;
  int Td;         // depths d >= Td are sparse: per-item child logits instead of level tiles
  int pair_rows;  // binary compat / node-key trees: child rows +c, -c (one dot per node)
  float* logA;    // causal, sparse levels: (B, L, H, T + 1) boundary log-masses between the kernels
};

constexpr int kLevelCols = 256;          // child columns of one level pass
constexpr int kXS = kLevelCols + 4;      // padded row stride (floats) of the logit tile
constexpr float kLn2 = 0.69314718055994531f;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float clampf(float x, float m) { return fminf(fmaxf(x, -m), m); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Child-logit products of one pass: up to kLevelCols/16 column tiles, tile t
// being the 16 summary rows from row(t) (rows past a level's nodes are zero
// padding); X[q][16t + c] = q . C[row(t) + c] for all 64 queries of the
// workgroup.  Wave w computes tiles w, w+4, ...; the next tile's summary
// fragments are loaded while the current tile's MFMAs run, and the first
// tile of the next pass is loaded (prefetch) before the caller consumes the
// current one.
template <typename E, int D, bool kLo>
struct LogitPipe {
  using M = Mfma<E>;
  using F = typename M::frag;
  static constexpr int KS = D / M::K;
  F ah[KS], al[KS];
  int64_t rmax;  // last valid summary row: tile rows past it read it (results unused)

  __device__ __forceinline__ void load(const E* hi, const E* lo, int64_t row, int lane, F (&h)[KS], F (&l)[KS]) {
    const int64_t r = min(row + (lane & 15), rmax);
    const int64_t rb = r * D + M::KPL * (lane >> 4);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      h[ks] = ld_frag(hi + rb + ks * M::K);
      if constexpr (kLo) l[ks] = ld_frag(lo + rb + ks * M::K);
    }
  }

  template <class RowFn>
  __device__ __forceinline__ void prefetch(const E* hi, const E* lo, RowFn row, int ntiles, int lane, int w) {
    if (w < ntiles) load(hi, lo, row(w), lane, ah, al);
  }

  template <int kStride, class RowFn>
  __device__ __forceinline__ void run(const RowFrags<E, D> (&qa)[4], float* Xs, const E* hi, const E* lo, RowFn row,
                                      int ntiles, int lane, int w) {
    const int col = lane & 15, g = lane >> 4;
    for (int ct = w; ct < ntiles; ct += 4) {
      F nh[KS], nl[KS];
      if (ct + 4 < ntiles) load(hi, lo, row(ct + 4), lane, nh, nl);
#pragma unroll
      for (int qt = 0; qt < 4; ++qt) {
        f32x4 c = zero4();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          c = M::mma(ah[ks], qa[qt].f[ks], c);
          if constexpr (kLo) c = M::mma(al[ks], qa[qt].f[ks], c);
        }
        *(f32x4*)(Xs + (16 * qt + col) * kStride + 16 * ct + 4 * g) = c;
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        ah[ks] = nh[ks];
        if constexpr (kLo) al[ks] = nl[ks];
      }
    }
  }
};

// The passes of one workgroup, in order: causal boundary batches (the
// boundary-path children of every depth, 16 column tiles per batch), then
// every level in chunks of kLevelCols children (causal: only children of
// nodes that contain a reachable leaf block).
struct Passes {
  int T, lb, causal, blk_lo, blk_hi, nbt;  // nbt: causal boundary tiles
  const Geo* G;
  int64_t base;                             // first summary row of this (batch, head)

  // depth d's boundary children: columns [c0, c0 + ncols) of level d + 1
  __device__ __forceinline__ int bc0(int d) const { return (blk_lo >> (lb * (T - d))) << lb; }
  __device__ __forceinline__ int bcols(int d) const {
    const int sh = lb * (T - d);
    return ((blk_hi >> sh) - (blk_lo >> sh) + 1) << lb;
  }
  __device__ __forceinline__ int btiles(int d) const { return (bcols(d) + 15) >> 4; }
  __device__ __forceinline__ int level_cols(int d) const {
    int n = G->pw[d + 1];
    if (causal) n = min(n, ((blk_hi >> (lb * (T - d))) + 1) << lb);
    return n;
  }
  __device__ __forceinline__ int nbatch(int cols) const { return (nbt + cols / 16 - 1) / (cols / 16); }
  // summary row of global boundary tile t
  __device__ __forceinline__ int64_t brow(int t) const {
    int d = 0, t0 = 0;
    while (t >= t0 + btiles(d)) {
      t0 += btiles(d);
      ++d;
    }
    return base + G->off[d + 1] + bc0(d) + 16 * (t - t0);
  }
};

// Uniform `idx` of the (B, L, H, S, T, b) tensor: from the caller's tensor,
// else word idx%4 of Philox(idx/4).  The last Philox block is cached per item.
struct RngCache {
  uint64_t ctr;
  uint32_t w0, w1, w2, w3;
};

__device__ __forceinline__ float uniform_at(const float* U, uint64_t seed, int64_t idx, RngCache& rc) {
  if (U) return U[idx];
  const uint64_t ctr = (uint64_t)idx >> 2;
  if (ctr != rc.ctr) {
    const Philox4 ph = philox4x32_10(ctr, seed);
    rc.ctr = ctr;
    rc.w0 = ph.w[0]; rc.w1 = ph.w[1]; rc.w2 = ph.w[2]; rc.w3 = ph.w[3];
  }
  const int wi = (int)(idx & 3);
  return word_to_uniform(wi == 0 ? rc.w0 : wi == 1 ? rc.w1 : wi == 2 ? rc.w2 : rc.w3);
}

// Lane (i - R) mod 16 of the same 16-lane row: a DPP row_ror.
template <int R>
__device__ __forceinline__ int row_ror(int x) {
  return __builtin_amdgcn_update_dpp(0, x, 0x120 + R, 0xf, 0xf, false);
}
template <int R>
__device__ __forceinline__ float row_ror(float x) {
  return __int_as_float(row_ror<R>(__float_as_int(x)));
}
__device__ __forceinline__ float row_max16(float x) {
  x = fmaxf(x, row_ror<8>(x));
  x = fmaxf(x, row_ror<4>(x));
  x = fmaxf(x, row_ror<2>(x));
  return fmaxf(x, row_ror<1>(x));
}
__device__ __forceinline__ float row_sum16(float x) {
  x += row_ror<8>(x);
  x += row_ror<4>(x);
  x += row_ror<2>(x);
  return x + row_ror<1>(x);
}
// Over the other lanes j of the row (j = s - R mod 16, earlier than s when
// R <= s): fst is cleared if an earlier lane holds the same leaf, and tot
// adds e of the later lanes with the same leaf.
template <int R = 1>
__device__ __forceinline__ void row_dups16(int n, float e, int s, float& tot, bool& fst) {
  if constexpr (R < 16) {
    const int nr = row_ror<R>(n);
    const float er = row_ror<R>(e);
    if (nr == n) {
      if (R <= s) fst = false;
      else tot += er;
    }
    row_dups16<R + 1>(n, e, s, tot, fst);
  }
}
// Lane j of each 16-lane row holds p[m] = its part of item m's sum (m < 16);
// returns item j's total (sum over the row's lanes of p[j]), by halving
// exchanges with lanes j ^ 8, j ^ 4, j ^ 2, j ^ 1.
__device__ __forceinline__ float row_reduce_scatter16(const float (&p)[16], int j) {
  float v8[8], v4[4], v2[2];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bool up = j & 8;
    v8[i] = (up ? p[i + 8] : p[i]) + row_xor<8>(up ? p[i] : p[i + 8], j);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool up = j & 4;
    v4[i] = (up ? v8[i + 4] : v8[i]) + row_xor<4>(up ? v8[i] : v8[i + 4], j);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const bool up = j & 2;
    v2[i] = (up ? v4[i + 2] : v4[i]) + row_xor<2>(up ? v4[i] : v4[i + 2], j);
  }
  const bool up = j & 1;
  return (up ? v2[1] : v2[0]) + row_xor<1>(up ? v2[0] : v2[1], j);
}

// rank = number of row keys below n; cnt = number of row keys that are not
// INT_MAX (this lane's included).
template <int R = 0>
__device__ __forceinline__ void row_rank16(int key, int n, int& rank, int& cnt) {
  if constexpr (R < 16) {
    const int kr = R == 0 ? key : row_ror<R>(key);
    rank += kr < n;
    cnt += kr != 0x7fffffff;
    row_rank16<R + 1>(key, n, rank, cnt);
  }
}

// Per-thread state of the root-to-leaf walks.  Items i = tid + 256 k map to
// (query i / S, sample i % S); each item's node, log-prob, causal boundary leaf
// block, uniforms' base index and (binary trees) last Philox block stay in
// registers.  decide() takes one decision from the node's child logits,
// finish() writes the weights and distinct leaf blocks; the dense-level kernel
// and the sparse-level kernel share both.
template <int kB, int kNI, bool kReplay>
struct Walk {
  // Per item: its node, (query << 8) | sample (query kQueryTile: inactive),
  // causal boundary leaf block, log-prob and, for b = 2 (two decisions per
  // Philox block), the block's last two words with the block's counter as
  // the tag: entered at word 0, a block serves the next decision from there.
  // The uniforms' index is recomputed from ub0 (the tile's first query and
  // sample) per decision, so few registers hold an item.
  static constexpr int kNC = kB == 2 ? kNI : 1;
  int node[kNI], qs[kNI], iblk[kNI];
  uint32_t rleaf[kReplay ? kNI : 1];  // replay: the given leaf block of each item
  float acc[kNI];
  uint32_t rtag[kNC], rw2[kNC], rw3[kNC];
  int64_t ub0;  // uniforms' (b, l, h, s) row of the tile's first query, sample 0

  __device__ __forceinline__ int iq(int k) const { return qs[k] >> 8; }
  __device__ __forceinline__ int is(int k) const { return qs[k] & 255; }

  __device__ __forceinline__ void init(const SampleArgs& a, int l0, int nq, int bb, int h, int tid) {
    const Geo& G = a.geo;
    const int S = a.S;
    const int nitems = kQueryTile * S;
    ub0 = (((int64_t)bb * a.L + l0) * a.H + h) * a.stot + a.s0;
#pragma unroll
    for (int k = 0; k < kNI; ++k) {
      const int it = tid + 256 * k;
      node[k] = 0;
      acc[k] = 0.f;
      int q = it < nitems ? it / S : kQueryTile;
      const int sm = it < nitems ? it - q * S : 0;
      if (q >= nq) q = kQueryTile;  // inactive item
      qs[k] = (q << 8) | sm;
      const int l = l0 + min(q, nq - 1);
      iblk[k] = (l + a.coff) / G.LB;
      if constexpr (kReplay) {
        rleaf[k] = 0u;
        if (q < kQueryTile)
          rleaf[k] = path_leaf(a.paths + ((((int64_t)l * a.B + bb) * a.H + h) * a.stot + a.s0 + sm) * a.nbytes,
                               a.nbits, a.nbytes);
      }
    }
#pragma unroll
    for (int k = 0; k < kNC; ++k) rtag[k] = rw2[k] = rw3[k] = 0u;
  }

  // One decision of item k at depth d from its node's b child logits xr[0..b)
  // (LDS for the dense passes, registers for the sparse levels); logA: the
  // causal boundary log-masses [64][T+1].
  __device__ __forceinline__ void decide(const SampleArgs& a, const float* logA, int k, int d, const float* xr) {
    const Geo& G = a.geo;
    const int T = G.T, lb = G.lb;
    const int b = kB ? kB : G.b;
    const int qi = iq(k);
    const int shb = lb * (T - d), shc = lb * (T - 1 - d);
    // log-sum-exp of the clamped child logits
    float lse;
    float x[kB ? kB : 1], ex[kB ? kB : 1];
    if constexpr (kB != 0) {
      float mx = -__builtin_inff();
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        x[j] = clampf(xr[j], a.maxhalf);
        mx = fmaxf(mx, x[j]);
      }
      float se = 0.f;
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        ex[j] = fast_exp2((x[j] - mx) * kLog2e);
        se += ex[j];
      }
      lse = mx + fast_log2(se) * kLn2;
    } else {
      float mx = -__builtin_inff();
      for (int j = 0; j < b; ++j) mx = fmaxf(mx, clampf(xr[j], a.maxhalf));
      float se = 0.f;
      for (int j = 0; j < b; ++j) se += fast_exp2((clampf(xr[j], a.maxhalf) - mx) * kLog2e);
      lse = mx + fast_log2(se) * kLn2;
    }
    if constexpr (kReplay) {  // the given digit, its log-prob (non-causal)
      const int jr = (int)((rleaf[k] >> (lb * (T - 1 - d))) & (uint32_t)(b - 1));
      float xj = 0.f;
      if constexpr (kB != 0) {
#pragma unroll
        for (int j = 0; j < kB; ++j)
          if (j == jr) xj = x[j];
      } else {
        xj = clampf(xr[jr], a.maxhalf);
      }
      node[k] = (node[k] << lb) + jr;
      acc[k] += xj - lse;
      return;
    }
    bool onb = false;
    int js = 0;
    float la_d = 0.f, la_c = 0.f;
    if (a.causal && (iblk[k] >> shb) == node[k]) {
      onb = true;
      js = (iblk[k] >> shc) & (b - 1);
      la_d = logA[qi * (T + 1) + d];
      la_c = logA[qi * (T + 1) + d + 1];
    }
    // index of the decision's first uniform in (B, L, H, stot, T, b)
    const int64_t ub = ((ub0 + (int64_t)qi * a.H * a.stot + is(k)) * T + d) * b;
    if constexpr (kB != 0) {
      // Gumbel-max in ratio form: lp_j - ln(-ln u_j) is, up to constants
      // common to all children, ln(p_j / E_j) with E_j = -log2 u_j > 0,
      // so the argmax is that of ex_j / E_j (ex_j = 2^((x_j - max) log2 e),
      // proportional to p_j); on the boundary the allowed weights are
      // ex_j (j < j*) and ex_j* A_{d+1}, rescaled to their own maximum.
      float u[kB];
      if constexpr (kB == 4) {  // the decision's four uniforms are one Philox block
        if (a.U) {
#pragma unroll
          for (int j = 0; j < 4; ++j) u[j] = a.U[ub + j];
        } else {
          const Philox4 ph = philox4x32_10((uint64_t)ub >> 2, a.seed);
#pragma unroll
          for (int j = 0; j < 4; ++j) u[j] = word_to_uniform(ph.w[j]);
        }
      } else {  // b = 2: ub is even, so the decision takes words 0, 1 or 2, 3 of a block
        if (a.U) {
          u[0] = a.U[ub];
          u[1] = a.U[ub + 1];
        } else {
          const uint64_t ctr = (uint64_t)ub >> 2;
          const bool hi = ub & 2;
          // rtag holds ctr + 1 of the block entered at word 0 (0: none), so a
          // fresh item never matches
          if (hi && rtag[k] == (uint32_t)ctr + 1u) {
            u[0] = word_to_uniform(rw2[k]);
            u[1] = word_to_uniform(rw3[k]);
          } else {
            const Philox4 ph = philox4x32_10(ctr, a.seed);
            u[0] = word_to_uniform(hi ? ph.w[2] : ph.w[0]);
            u[1] = word_to_uniform(hi ? ph.w[3] : ph.w[1]);
            rtag[k] = hi ? 0u : (uint32_t)ctr + 1u;
            rw2[k] = ph.w[2];
            rw3[k] = ph.w[3];
          }
        }
      }
      float wj[kB];
#pragma unroll
      for (int j = 0; j < kB; ++j) wj[j] = ex[j];
      if (onb) {
        float y[kB], my = -__builtin_inff();
#pragma unroll
        for (int j = 0; j < kB; ++j) {
          y[j] = j < js ? x[j] * kLog2e : j == js ? x[j] * kLog2e + la_c * kLog2e : -__builtin_inff();
          my = fmaxf(my, y[j]);
        }
#pragma unroll
        for (int j = 0; j < kB; ++j) wj[j] = j <= js ? fast_exp2(y[j] - my) : 0.f;
      }
      float bw = wj[0], be = -fast_log2(u[0]);
      int bj = 0;
#pragma unroll
      for (int j = 1; j < kB; ++j) {
        const float e = -fast_log2(u[j]);
        if (wj[j] * be > bw * e) {
          bw = wj[j];
          be = e;
          bj = j;
        }
      }
      float xb_ = x[0];
#pragma unroll
      for (int j = 1; j < kB; ++j)
        if (j == bj) xb_ = x[j];
      float lp = xb_ - lse;
      if (onb) lp += bj < js ? -la_d : la_c - la_d;
      node[k] = (node[k] << lb) + bj;
      acc[k] += lp;
      return;
    }
    RngCache local;
    local.ctr = ~0ull;
    local.w0 = local.w1 = local.w2 = local.w3 = 0u;
    RngCache& cache = local;
    float best = -__builtin_inff(), bl = 0.f;
    int bj = 0;
    auto consider = [&](int j, float xj) {
      float lp = xj - lse;
      if (onb) {
        if (j < js) lp -= la_d;
        else if (j == js) lp += la_c - la_d;
        else lp = -__builtin_inff();
      }
      const float u = uniform_at(a.U, a.seed, ub + j, cache);
      // lp + g up to the common constant -log(ln 2): g = -ln(ln2 * -log2 u)
      const float sc = lp - kLn2 * fast_log2(-fast_log2(u));
      if (sc > best) {
        best = sc;
        bj = j;
        bl = lp;
      }
    };
    for (int j = 0; j < b; ++j) consider(j, clampf(xr[j], a.maxhalf));
    node[k] = (node[k] << lb) + bj;
    acc[k] += bl;
  }

  // The walk's state between the dense-level and the sparse-level kernels:
  // node and log-prob per item (in the record's leaf / slot-weight arrays,
  // which finish() overwrites) and, causal, the boundary log-masses.
  __device__ __forceinline__ void save(const SampleArgs& a, const float* logA, int l0, int nq, int bb, int h,
                                       int tid) {
    const int S = a.S, T1 = a.geo.T + 1;
#pragma unroll
    for (int k = 0; k < kNI; ++k) {
      if (iq(k) >= kQueryTile) continue;
      const int64_t o = (((int64_t)bb * a.L + l0 + iq(k)) * a.H + h) * S + is(k);
      a.leaf[o] = node[k];
      a.slot_weight[o] = acc[k];
    }
    if (a.causal)
      for (int e = tid; e < nq * T1; e += 256) {
        const int qi = e / T1, d = e - qi * T1;
        a.logA[(((int64_t)bb * a.L + l0 + qi) * a.H + h) * T1 + d] = logA[qi * T1 + d];
      }
  }
  __device__ __forceinline__ void load(const SampleArgs& a, float* logA, int l0, int nq, int bb, int h, int tid) {
    const int S = a.S, T1 = a.geo.T + 1;
#pragma unroll
    for (int k = 0; k < kNI; ++k) {
      if (iq(k) >= kQueryTile) continue;
      const int64_t o = (((int64_t)bb * a.L + l0 + iq(k)) * a.H + h) * S + is(k);
      node[k] = a.leaf[o];
      acc[k] = a.slot_weight[o];
    }
    if (a.causal)
      for (int e = tid; e < nq * T1; e += 256) {
        const int qi = e / T1, d = e - qi * T1;
        logA[qi * T1 + d] = a.logA[(((int64_t)bb * a.L + l0 + qi) * a.H + h) * T1 + d];
      }
  }

  // Weights (softmax over the query's samples) and distinct leaf blocks;
  // Xs: LDS scratch of at least 3 * 64 * S words.
  __device__ __forceinline__ void finish(const SampleArgs& a, float* Xs, int l0, int bb, int h, int tid) {
    const int S = a.S;
    const int lane = tid & 63;
    const int nitems = kQueryTile * S;
    int* lf = (int*)Xs;
    float* lps = Xs + kQueryTile * S;
    int* fl = (int*)(Xs + 2 * kQueryTile * S);
    // weights (softmax over the query's samples) and distinct leaf blocks
    if (S == 16) {
      // item tid + 256 k: a query's 16 samples are the 16 lanes of one DPP row
      const int s = lane & 15;
  #pragma unroll
      for (int k = 0; k < kNI; ++k) {
        const float m = row_max16(acc[k]);
        const float e = fast_exp2((acc[k] - m) * kLog2e);
        const float se = row_sum16(e);
        const float inv = 1.f / se;
        float tot = e;  // weight of this leaf block summed over the samples from s on
        bool fst = true;
        row_dups16(node[k], e, s, tot, fst);
        int rank = 0, cnt = 0;
        row_rank16(fst ? node[k] : 0x7fffffff, node[k], rank, cnt);
        const int qi = iq(k);
        if (qi >= kQueryTile) continue;
        const int l = l0 + qi;
        const int64_t qh = ((int64_t)bb * a.L + l) * a.H + h;
        a.weights[bb * a.wsb + (int64_t)l * a.wsl + h * a.wsh + s] = e * inv;
        a.leaf[qh * S + s] = node[k];
        if (fst) {
          a.slot_leaf[qh * S + rank] = node[k];
          a.slot_weight[qh * S + rank] = tot * inv;
        }
        if (s == 0) {
          a.slot_count[qh] = cnt;
          a.lse[qh] = m + fast_log2(se) * kLn2;
        }
      }
      return;
    }
  #pragma unroll
    for (int k = 0; k < kNI; ++k) {
      const int it = tid + 256 * k;
      if (it < nitems) {
        lf[it] = node[k];
        lps[it] = acc[k];
      }
    }
    __syncthreads();
    float wgt[kNI];
    bool first[kNI];
  #pragma unroll
    for (int k = 0; k < kNI; ++k) {
      wgt[k] = 0.f;
      first[k] = false;
      const int qi = iq(k);
      if (qi >= kQueryTile) continue;
      const int s = is(k);
      const int* lq = lf + qi * S;
      const float* pq = lps + qi * S;
      float m = -__builtin_inff();
      for (int j = 0; j < S; ++j) m = fmaxf(m, pq[j]);
      float sum = 0.f, tot = 0.f;
      bool fst = true;
      for (int j = 0; j < S; ++j) {
        const float e = fast_exp2((pq[j] - m) * kLog2e);
        sum += e;
        if (lq[j] == node[k]) {
          if (j < s) fst = false;
          else tot += e;
        }
      }
      const float inv = 1.f / sum;
      if (s == 0) a.lse[(((int64_t)bb * a.L + l0 + qi) * a.H + h)] = m + fast_log2(sum) * kLn2;
      wgt[k] = fast_exp2((acc[k] - m) * kLog2e) * inv;
      first[k] = fst;
      acc[k] = tot * inv;  // summed weight of this leaf block (used if first)
    }
    // distinct-leaf keys: the leaf for a first occurrence, else INT_MAX
  #pragma unroll
    for (int k = 0; k < kNI; ++k) {
      const int it = tid + 256 * k;
      if (iq(k) < kQueryTile) fl[it] = first[k] ? node[k] : 0x7fffffff;
      else if (it < nitems) fl[it] = 0x7fffffff;
    }
    __syncthreads();
  #pragma unroll
    for (int k = 0; k < kNI; ++k) {
      const int qi = iq(k);
      if (qi >= kQueryTile) continue;
      const int s = is(k);
      const int l = l0 + qi;
      const int64_t qh = ((int64_t)bb * a.L + l) * a.H + h;
      a.weights[bb * a.wsb + (int64_t)l * a.wsl + h * a.wsh + s] = wgt[k];
      a.leaf[qh * S + s] = node[k];
      const int* fq = fl + qi * S;
      if (first[k]) {
        int rank = 0;
        for (int j = 0; j < S; ++j) rank += fq[j] < node[k];
        a.slot_leaf[qh * S + rank] = node[k];
        a.slot_weight[qh * S + rank] = acc[k];
      }
      if (s == 0) {
        int cnt = 0;
        for (int j = 0; j < S; ++j) cnt += fq[j] != 0x7fffffff;
        a.slot_count[qh] = cnt;
      }
    }
  }
};

// kB: branching known at compile time (2 or 4), or 0 for the runtime value.
// kNI: (query, sample) items per thread, >= 64 * S / 256.
// kReplay: decisions come from a.paths (packed path bits) instead of Gumbel-max.
template <typename E, int D, int kB, int kNI, bool kReplay, int kC>
// Binary trees with 16 items per thread at head dims of 96 and up spill at
// two waves per SIMD; one wave with the whole register file runs them faster
// (the reference tree at L = 16384, 64 paths: 5.85 -> 4.14 ms; branching 4
// is faster at two waves).
__global__ __launch_bounds__(256, (kB == 2 && kNI >= 16 && D >= 96) ? 1 : kC < kLevelCols ? 3 : 2) void sample_kernel(SampleArgs a) {
  extern __shared__ __align__(16) char smem[];
  const Geo& G = a.geo;
  const int bh = blockIdx.y, bb = bh / a.H, h = bh - bb * a.H;
  const int l0 = blockIdx.x * kQueryTile;
  const int nq = min(kQueryTile, a.L - l0);
  const int S = a.S, T = G.T, lb = G.lb;
  const int b = kB ? kB : G.b;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t rows = G.NS;
  constexpr bool kLo = sizeof(E) == 2;

  float* Xs = (float*)smem;                      // [64][(kC + 4)] logits of one level pass
  float* logA = Xs + kQueryTile * (kC + 4);           // [64][T+1] causal boundary log-mass
  float* xb = logA + kQueryTile * (T + 1);       // [64][T*b] boundary child logits
  // after the walk Xs is reused by finish()

  // all 64 query rows as MFMA B fragments (rows past nq are zero)
  RowFrags<E, D> qa[4];
#pragma unroll
  for (int qt = 0; qt < 4; ++qt) {
    const int r = 16 * qt + (lane & 15);
    qa[qt].load(r < nq ? (const E*)a.q + bb * a.qsb + (int64_t)(l0 + r) * a.qsl + h * a.qsh : nullptr, lane >> 4);
  }
  const E* hi = (const E*)(sizeof(E) == 2 ? a.sum_hi : (const void*)a.sum32);
  const E* lo = (const E*)a.sum_lo;

  Passes ps;
  ps.T = T;
  ps.lb = lb;
  ps.causal = a.causal && T > 0;
  // leaf blocks [0, blk_hi] are reachable from some query of the tile
  ps.blk_lo = (l0 + a.coff) / G.LB;
  ps.blk_hi = (l0 + nq - 1 + a.coff) / G.LB;
  ps.G = &G;
  ps.base = (int64_t)bh * rows;
  ps.nbt = 0;
  if (ps.causal)
    for (int d = 0; d < T; ++d) ps.nbt += ps.btiles(d);
  const int nbatch = ps.causal ? ps.nbatch(kC) : 0;

  Walk<kB, kNI, kReplay> wk;
  wk.init(a, l0, nq, bb, h, tid);

  // pass p < nbatch: causal boundary batch p; then level d, chunk c0
  LogitPipe<E, D, kLo> pipe;
  pipe.rmax = ps.base + rows - 1;
  auto tiles_of = [&](int p, int d, int c0) {
    if (p < nbatch) return min(kC / 16, ps.nbt - p * (kC / 16));
    return (min(kC, ps.level_cols(d) - c0) + 15) >> 4;
  };
  auto prefetch = [&](int p, int d, int c0) {
    if (p < nbatch) {
      const int t0 = p * (kC / 16);
      pipe.prefetch(hi, lo, [&](int t) { return ps.brow(t0 + t); }, tiles_of(p, d, c0), lane, w);
    } else {
      const int64_t r0 = ps.base + G.off[d + 1] + c0;
      pipe.prefetch(hi, lo, [&](int t) { return r0 + 16 * t; }, tiles_of(p, d, c0), lane, w);
    }
  };
  // A level wider than kC children takes several passes, run from the
  // highest column chunk down: an item that moves in the pass at c0 lands on a
  // node >= c0 of the next depth, whose children (>= 2 c0) lie past every
  // later pass of the level, so no item decides twice in one level.
  auto last_c0 = [&](int dd) { return (ps.level_cols(dd) - 1) / kC * kC; };
  const int Td = a.Td;  // dense levels 0 .. Td - 1
  int p = 0, d = 0, c0 = 0;  // current pass (level 0 has b <= kC children)
  if (nbatch > 0 || Td > 0) prefetch(0, 0, 0);
  while (p < nbatch || d < Td) {
    const int nt = tiles_of(p, d, c0);
    if (p < nbatch) {
      const int t0 = p * (kC / 16);
      pipe.template run<kC + 4>(qa, Xs, hi, lo, [&](int t) { return ps.brow(t0 + t); }, nt, lane, w);
    } else {
      const int64_t r0 = ps.base + G.off[d + 1] + c0;
      pipe.template run<kC + 4>(qa, Xs, hi, lo, [&](int t) { return r0 + 16 * t; }, nt, lane, w);
    }
    __syncthreads();
    // next pass, and its first tile in flight while this one is consumed
    int np = p + 1, nd = d, nc0 = c0;
    if (p >= nbatch) {
      if (c0 > 0) {
        nc0 = c0 - kC;
      } else {
        ++nd;
        nc0 = nd < Td ? last_c0(nd) : 0;
      }
    }
    if (np < nbatch || nd < Td) prefetch(np, nd, nc0);

    if (p < nbatch) {
      // boundary child logits of this batch's depths: query tid & 63, depths
      // w, w + 4, ... (all four waves)
      const int qb = tid & 63;
      if (qb < nq) {
        const int blk = (l0 + qb + a.coff) / G.LB;
        int t0 = 0;
        for (int dd = 0; dd < T; ++dd) {
          // column of the query's boundary node's first child in the global tile space
          const int gc = 16 * t0 + ((blk >> (lb * (T - dd))) << lb) - ps.bc0(dd) - p * kC;
          if ((dd & 3) == w && gc >= 0 && gc < kC)
            for (int j = 0; j < b; ++j) xb[qb * T * b + dd * b + j] = clampf(Xs[qb * (kC + 4) + gc + j], a.maxhalf);
          t0 += ps.btiles(dd);
        }
      }
      if (p + 1 == nbatch) {
        // Causal: allowed log-mass of each boundary-path node, bottom-up:
        // A_T = 1, A_d = sum_{j<j*} p_j + p_{j*} A_{d+1}.  Per depth (waves
        // split the depths), in log2 units: lt = log2 sum_{j<j*} p_j and
        // lj = log2 p_{j*}, written over the depth's first two logits.
        __syncthreads();
        if (qb < nq) {
          const int blk = (l0 + qb + a.coff) / G.LB;
          for (int dd = w; dd < T; dd += 4) {
            const int js = (blk >> (lb * (T - 1 - dd))) & (b - 1);
            float* xs = xb + qb * T * b + dd * b;
            float mx = -__builtin_inff(), ml = -__builtin_inff();
            for (int j = 0; j < b; ++j) {
              mx = fmaxf(mx, xs[j]);
              if (j < js) ml = fmaxf(ml, xs[j]);
            }
            float se = 0.f, sl = 0.f;
            for (int j = 0; j < b; ++j) {
              se += fast_exp2((xs[j] - mx) * kLog2e);
              if (j < js) sl += fast_exp2((xs[j] - ml) * kLog2e);
            }
            const float l2se = fast_log2(se);
            const float lj = (xs[js] - mx) * kLog2e - l2se;
            const float lt = js > 0 ? (ml - mx) * kLog2e + fast_log2(sl) - l2se : -__builtin_inff();
            xs[0] = lt;
            xs[1] = lj;
          }
        }
        __syncthreads();
        if (tid < nq) {
          float* la = logA + tid * (T + 1);
          const float* xq = xb + tid * T * b;
          float c = 0.f;  // log2 A_{d+1}
          la[T] = 0.f;
          for (int dd = T - 1; dd >= 0; --dd) {
            const float lt = xq[dd * b], v = xq[dd * b + 1] + c;
            const float hi = fmaxf(lt, v), lo = fminf(lt, v);
            c = hi + fast_log2(1.f + fast_exp2(lo - hi));
            la[dd] = c * kLn2;
          }
        }
      }
    } else {
      const int ncols = min(kC, ps.level_cols(d) - c0);
#pragma unroll
      for (int k = 0; k < kNI; ++k) {
        const int qi = wk.iq(k);
        if (qi >= kQueryTile) continue;
        const int base = (wk.node[k] << lb) - c0;
        if (base < 0 || base >= ncols) continue;
        wk.decide(a, logA, k, d, Xs + qi * (kC + 4) + base);
      }
    }
    __syncthreads();
    p = np;
    d = nd;
    c0 = nc0;
  }


  if (Td < T) {  // the sparse-level kernel continues the walks
    wk.save(a, logA, l0, nq, bb, h, tid);
    return;
  }
  wk.finish(a, Xs, l0, bb, h, tid);
}

// The sparse levels (d >= Td, wider than level tiles pay for), continuing the
// walks the dense-level kernel saved: each item's child logits are dot
// products of its query row with its node's child summary rows (float).  The
// 16 lanes of a DPP row take the row's 16 items in turn, lane j covering head
// dims [DPL j, DPL (j + 1)) (one coalesced 16 * DPL-float piece of the
// summary row per item), then a reduce-scatter over the row leaves each lane
// its own item's logits.  Cost per item and level: b summary rows (compat /
// node-key trees: 1), linear in L.  Same grid and LDS as sample_kernel.
template <typename E, int D, int kB, int kNI, bool kReplay>
__global__ __launch_bounds__(256) void sample_sparse_kernel(SampleArgs a) {
  static_assert(kB == 2 || kB == 4, "sparse levels: b = 2 or 4");
  extern __shared__ __align__(16) char smem[];
  const Geo& G = a.geo;
  const int bh = blockIdx.y, bb = bh / a.H, h = bh - bb * a.H;
  const int l0 = blockIdx.x * kQueryTile;
  const int nq = min(kQueryTile, a.L - l0);
  const int T = G.T, Td = a.Td;
  const int tid = threadIdx.x, lane = tid & 63;
  float* Xs = (float*)smem;                 // [64][D + 4] query rows, then finish()'s arrays
  float* logA = Xs + kQueryTile * kXS;      // [64][T+1]
  Walk<kB, kNI, kReplay> wk;
  wk.init(a, l0, nq, bb, h, tid);
  wk.load(a, logA, l0, nq, bb, h, tid);
  {
    constexpr int QS = D + 4;
    float* qs = Xs;  // [64][QS] float query rows (the logit tile is free now)
    for (int e = tid; e < kQueryTile * (D / 8); e += 256) {
      const int r = e / (D / 8), c = (e - r * (D / 8)) * 8;
      float v8[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v8[i] = 0.f;
      if (r < nq) {
        const E* src = (const E*)a.q + bb * a.qsb + (int64_t)(l0 + r) * a.qsl + h * a.qsh + c;
#pragma unroll
        for (int i = 0; i < 8; ++i) v8[i] = tof(src[i]);
      }
      *(float4*)(qs + r * QS + c) = make_float4(v8[0], v8[1], v8[2], v8[3]);
      *(float4*)(qs + r * QS + c + 4) = make_float4(v8[4], v8[5], v8[6], v8[7]);
    }
    __syncthreads();
    constexpr int DPL = D / 16;  // head dims per lane: 2, 4, 6 or 8
    const int j16 = lane & 15, r0 = lane & 48;
    const int nrow = a.pair_rows ? 1 : kB;
    // each wave's items (query, node) in LDS past the query rows, so a row's
    // 16 lanes read item m with one broadcast load; a wave reads only its own
    // entries, which LDS orders after its writes
    static_assert(kQueryTile * (D + 4) * 4 + 4 * kNI * 64 * 8 <= kQueryTile * kXS * 4, "item table fits");
    int2* tab = (int2*)(qs + kQueryTile * QS) + (tid >> 6) * kNI * 64;
    for (int dd = Td; dd < T; ++dd) {
      const float* lvl = a.sum32 + ((int64_t)bh * G.NS + G.off[dd + 1]) * D + DPL * j16;
#pragma unroll
      for (int k = 0; k < kNI; ++k) tab[k * 64 + lane] = make_int2(wk.iq(k), wk.node[k]);
#pragma unroll
      for (int k = 0; k < kNI; ++k) {
        float part[kB][16];
#pragma unroll
        for (int m = 0; m < 16; ++m) {
          const int2 it = tab[k * 64 + r0 + m];
          const int qm = it.x, nm = it.y;
          const bool act = qm < kQueryTile;
          const float* qrow = qs + (act ? qm : 0) * QS + DPL * j16;
          float qv[DPL];
#pragma unroll
          for (int i = 0; i < DPL; i += 2) {
            const float2 t = *(const float2*)(qrow + i);
            qv[i] = t.x;
            qv[i + 1] = t.y;
          }
#pragma unroll
          for (int j = 0; j < kB; ++j) {
            float sacc = 0.f;
            if (j < nrow) {
              const float* crow = lvl + ((int64_t)(act ? nm : 0) * kB + j) * D;
#pragma unroll
              for (int i = 0; i < DPL; i += 2) {
                const float2 t = *(const float2*)(crow + i);
                sacc += qv[i] * t.x + qv[i + 1] * t.y;
              }
            }
            part[j][m] = sacc;
          }
        }
        float xo[kB];
#pragma unroll
        for (int j = 0; j < kB; ++j) xo[j] = row_reduce_scatter16(part[j], j16);
        if (a.pair_rows) xo[1] = -xo[0];
        if (wk.iq(k) < kQueryTile) wk.decide(a, logA, k, dd, xo);
      }
    }
    __syncthreads();  // qs (Xs) is reused below
  }
  wk.finish(a, Xs, l0, bb, h, tid);
}

// Xs (which the final phase's three [64][S] arrays alias: 3 * 64 * 64 * 4
// bytes < sizeof Xs), logA and the boundary child logits.
static inline int sample_smem(const Plan& P, int cols) {
  const int T = P.geo.T, b = P.geo.b;
  return kQueryTile * (cols + 4) * 4 + kQueryTile * (T + 1) * 4 + kQueryTile * T * b * 4;
}

// Child columns per level pass of sample_kernel: 128 where that lets a third
// workgroup onto a CU (head dims up to 32, or 64 for 16-bit inputs, whose
// registers fit three waves per SIMD; up to 16 samples, whose final phase fits
// the smaller logit tile), else kLevelCols.
static inline int sample_cols(const Plan& P) {
  return (P.D <= 32 || (P.D <= 64 && P.esize == 2)) && P.S <= 16 && (P.geo.b == 2 || P.geo.b == 4) ? 128
                                                                                                   : kLevelCols;
}

template <bool kReplay, typename E, int D, int kB, int kNI>
static hipError_t sample_impl(const Plan& P, const void* q, const float* U, uint64_t seed, float* weights,
                              char* rec, hipStream_t st, const uint8_t* paths) {
  SampleArgs a;
  a.geo = P.geo;
  a.B = (int)P.B;
  a.paths = paths;
  a.nbits = P.geo.T * P.geo.lb;
  a.nbytes = (a.nbits + 7) / 8;
  a.L = (int)P.L;
  a.H = (int)P.H;
  a.S = (int)P.S;
  a.s0 = (int)P.s0;
  a.stot = (int)P.s_total;
  a.causal = P.p.causal == TA_CAUSAL_EXACT;
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
  a.lse = (float*)(rec + P.rec.lse);
  a.Td = P.sample_dense;
  a.pair_rows = P.p.tree_mode != TA_TREE_NATURAL && P.geo.b == 2;
  a.logA = (float*)(rec + P.rec.logA);
  auto launch = [&](auto kern, int smem) -> hipError_t {
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, smem);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3((unsigned)((P.L + kQueryTile - 1) / kQueryTile), P.BH), dim3(256), smem, st, a);
    return hipGetLastError();
  };
  hipError_t e;
  if constexpr ((kB == 2 || kB == 4) && (D <= 32 || (D <= 64 && sizeof(E) == 2)) && kNI == 4) {
    e = sample_cols(P) == 128 ? launch(sample_kernel<E, D, kB, kNI, kReplay, 128>, sample_smem(P, 128))
                              : launch(sample_kernel<E, D, kB, kNI, kReplay, kLevelCols>, sample_smem(P, kLevelCols));
  } else {
    e = launch(sample_kernel<E, D, kB, kNI, kReplay, kLevelCols>, sample_smem(P, kLevelCols));
  }
  if constexpr (kB == 2 || kB == 4)
    if (e == hipSuccess && P.sample_dense < P.geo.T)
      e = launch(sample_sparse_kernel<E, D, kB, kNI, kReplay>, sample_smem(P, kLevelCols));
  return e;
}

template <bool kReplay, typename E, int D>
static hipError_t sample_b(const Plan& P, const void* q, const float* U, uint64_t seed, float* w, char* rec,
                           hipStream_t st, const uint8_t* pa) {
  static_assert(kMaxSamples * kQueryTile / 256 == 16, "items per thread");
  // 64 * S / 256 items per thread: 4 (S <= 16), 8 (S <= 32) or 16
  const int ni = P.S <= 16 ? 4 : P.S <= 32 ? 8 : 16;
  switch (P.geo.b) {
    case 2: return ni == 4 ? sample_impl<kReplay, E, D, 2, 4>(P, q, U, seed, w, rec, st, pa)
                 : ni == 8 ? sample_impl<kReplay, E, D, 2, 8>(P, q, U, seed, w, rec, st, pa)
                           : sample_impl<kReplay, E, D, 2, 16>(P, q, U, seed, w, rec, st, pa);
    case 4: return ni == 4 ? sample_impl<kReplay, E, D, 4, 4>(P, q, U, seed, w, rec, st, pa)
                 : ni == 8 ? sample_impl<kReplay, E, D, 4, 8>(P, q, U, seed, w, rec, st, pa)
                           : sample_impl<kReplay, E, D, 4, 16>(P, q, U, seed, w, rec, st, pa);
    default: return ni == 4 ? sample_impl<kReplay, E, D, 0, 4>(P, q, U, seed, w, rec, st, pa)
                  : ni == 8 ? sample_impl<kReplay, E, D, 0, 8>(P, q, U, seed, w, rec, st, pa)
                            : sample_impl<kReplay, E, D, 0, 16>(P, q, U, seed, w, rec, st, pa);
  }
}

template <bool kReplay, typename E>
static hipError_t sample_d(const Plan& P, const void* q, const float* U, uint64_t seed, float* w, char* rec,
                           hipStream_t st, const uint8_t* pa) {
  switch (P.D) {
    case 32: return sample_b<kReplay, E, 32>(P, q, U, seed, w, rec, st, pa);
    case 64: return sample_b<kReplay, E, 64>(P, q, U, seed, w, rec, st, pa);
    case 96: return sample_b<kReplay, E, 96>(P, q, U, seed, w, rec, st, pa);
    default: return sample_b<kReplay, E, 128>(P, q, U, seed, w, rec, st, pa);
  }
}

// The sampler of one element type, every head dim and branching, with
// Gumbel-max decisions (kReplay false) or replayed paths (kReplay true); each
// (kReplay, E) is defined in a translation unit of its own (sample*.hip), so
// the six compile in parallel.
template <bool kReplay, typename E>
hipError_t sample_typed(const Plan& P, const void* q, const float* U, uint64_t seed, float* weights, char* rec,
                        hipStream_t st, const uint8_t* paths);
#define TA_SAMPLE_TYPED_DECL(R, E)                                                                             \
  template <>                                                                                                  \
  hipError_t sample_typed<R, E>(const Plan& P, const void* q, const float* U, uint64_t seed, float* weights, \
                                char* rec, hipStream_t st, const uint8_t* paths);
TA_SAMPLE_TYPED_DECL(false, float)
TA_SAMPLE_TYPED_DECL(false, bf16)
TA_SAMPLE_TYPED_DECL(false, f16)
TA_SAMPLE_TYPED_DECL(true, float)
TA_SAMPLE_TYPED_DECL(true, bf16)
TA_SAMPLE_TYPED_DECL(true, f16)
#undef TA_SAMPLE_TYPED_DECL

template <bool kReplay>
static hipError_t sample_dispatch(const Plan& P, const void* q, const float* U, uint64_t seed, float* weights,
                                  char* rec, hipStream_t st, const uint8_t* paths) {
  switch (P.p.dtype) {
    case TA_F32: return sample_typed<kReplay, float>(P, q, U, seed, weights, rec, st, paths);
    case TA_BF16: return sample_typed<kReplay, bf16>(P, q, U, seed, weights, rec, st, paths);
    default: return sample_typed<kReplay, f16>(P, q, U, seed, weights, rec, st, paths);
  }
}

#define TA_SAMPLE_TYPED(R, E)                                                                                    \
  template <>                                                                                                    \
  hipError_t sample_typed<R, E>(const Plan& P, const void* q, const float* U, uint64_t seed, float* weights,   \
                                char* rec, hipStream_t st, const uint8_t* paths) {                              \
    return sample_d<R, E>(P, q, U, seed, weights, rec, st, paths);                                               \
  }

}  // namespace ta
