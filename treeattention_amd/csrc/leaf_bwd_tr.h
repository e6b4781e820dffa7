// The 16-bit leaf backward (leaf_bwd_tr_kernel) and its arguments, shared by
// leaf_bwd.hip (the leaf part alone) and leaf_bwd_path.hip (with the tree
// gradient of every pair's sampled path), which compile in parallel.
//
// Path rows.  Every pair of a leaf block's bucket walked the same root path
// to the block, so its tree gradient needs only the T*b child summaries of
// that path (child j of the path node at depth d: row d*b + j), the same for
// the whole workgroup.  For a pair with summed weight W and leaf delta
// delta = dout . o, dl = W (delta - mean) with mean = dout . out over the
// query's samples, and at depth d with child probabilities p_j (softmax of
// the clamped logits x_j = q . c_j) the pair adds
//   gamma_j = dl ([j on the path] - p_j)      (0 where x_j was clamped)
// to the logit gradient of child j.  Summed over a query's pairs this is the
// reference's per-sample gradient (_autograd.py:789-856; the per-node sums
// A_row - p_j A_n are sums over the pairs below each node).  The kernel gets
//   X = C_path Q^T             (one more MFMA tile next to S = K Q^T),
//   dq_pair += gamma C_path     (gamma as extra key columns of dz),
//   dC_path += gamma^T Q        (extra key rows of the dK product),
// writes dC_path per leaf block, and the tree backward sums the blocks under
// each node (path_dsum_kernel) and the pairs' dq rows (dq_rows_kernel): no
// dense level tiles, no G^T rows, no per-sample log-prob gradients.
#pragma once

#include "launch.h"

namespace ta {

struct LeafBwdArgs {
  int B, L, N, H, S, NL, LB, causal;
  float scale, scale_log2;
  const void *q, *k, *v, *g;
  int64_t qsb, qsl, qsh, ksb, ksl, ksh, vsb, vsl, vsh, gsb, gsl, gsh;
  const int* order;
  const int* block_start;
  const float* slot_weight;
  float* delta;     // (B,L,H,S), or null
  void* dq_part;    // E (B,L,H,S,D)
  void* dv;         // E, v strides
  float* dk_leaf;   // (B,N,H,D) or null
  float* dv32;      // chunked problem: dv as float (B,N,H,D) rows, else null
  int first;        // chunked problem: the first chunk writes dv32 / dk_leaf, later ones add
  // path rows (leaf_bwd_path.hip)
  Geo geo;
  int NS;
  float maxhalf, inv_scale;
  const void* sum_hi;  // E (BH, NS, D) child summaries
  const float* mean;   // (B, L, H): dout . out over the query's samples
  float* dcp;          // (BH, NL, T*b, D): each block's gradient of its path's child summaries
};

// One element of the float accumulators of a chunked problem (or of dk_leaf).
__device__ __forceinline__ void acc1f(float* p, float x, int first) { *p = first ? x : *p + x; }

// Transposing-read variant for 16-bit inputs: eight waves and 128-pair tiles
// (four waves and 64-pair tiles for 128-key blocks).  Phase A (each wave,
// its 16 pairs): query and output-gradient rows come straight from global
// memory into MFMA fragments (the next tile's are loaded while this one
// computes), then P, delta, dz and the pair's dq; the wave then stores its
// rows of Q, dout, wP and dz into row-major LDS tiles with 16- and 8-byte
// writes.  Phase B (all waves, each a block of output tiles): dV += (wP)^T dout
// and dK += dz^T Q over the tile's pairs.  The MFMA operands of phase B and
// K^T of the dq product are read with ds_read_b64_tr_b16, gfx950's transposing
// LDS read: within each group of 16 lanes, lane i receives element i%4 of the
// 8-byte slots of lanes 4r + i/4 (r = 0..3), so pointing lane j of a group at
// row k0 + j/4, columns 4(j%4).. of a row-major [k][n] tile gives lane i the
// four values [k0..k0+3][n = i] -- a k-contiguous operand column.  Row strides
// are padded by 16 elements so every 16-lane group touches distinct banks.
// Eight waves.  Leaf blocks of up to 64 keys take 128-pair tiles, 16 pairs
// per wave; 128-key blocks (and 64-key blocks with 32 path rows at large
// head dims) take 64-pair tiles so the K / V, pair-row and P / dz tiles fit
// the LDS; their phase A runs on waves 0-3 while all eight share phase B.
// TR path rows (0, 16 or 32) add the [TR][RS] path summaries and TR key
// columns to the dz tile.
constexpr int bwd_tr_bytes(int D, int LBP, int TR, int QT) {
  return (2 * LBP * (D + 16) + 2 * QT * (D + 16) + QT * (LBP + 16) +
          QT * (LBP + TR + 16 + (((LBP + TR + 16) / 16) % 4 == 0 ? 16 : 0)) + TR * (D + 16)) * 2;
}
constexpr int bwd_tr_qt(int D, int LBP, int TR) {
  return LBP <= 64 && bwd_tr_bytes(D, LBP, TR, 128) <= 160 * 1024 ? 128 : 64;
}
template <int D, int LBP, int TR>
struct BwdTrTile {
  static constexpr int NW = 8;                      // waves
  static constexpr int QT = bwd_tr_qt(D, LBP, TR);  // pairs per tile, 16 per phase-A wave
  static constexpr int RS = D + 16, PS = LBP + 16;
  // dz rows: keys, then path rows; a stride of 16 x (not a multiple of 4)
  // elements keeps the transposing reads of four rows on distinct banks
  static constexpr int ZS = LBP + TR + 16 + (((LBP + TR + 16) / 16) % 4 == 0 ? 16 : 0);
  static constexpr int bytes = bwd_tr_bytes(D, LBP, TR, QT);
  // waves per SIMD the registers must allow: two workgroups per CU where the
  // LDS holds two (head dim 32 with 32-key blocks), else one
  static constexpr int MINW = 2 * bytes <= 160 * 1024 && D <= 32 && LBP <= 32 ? 4 : 2;
};

// One pair column's operands for a tile: query and output-gradient row
// fragments, the pair's summed sample weight, its query row (-1: padding),
// its (b, l, h, u) slot and (path rows) its query's dout . out.
template <typename E, int D>
struct PairRows {
  RowFrags<E, D> q, g;
  float w, mn;
  int l;
  int64_t sl;
  // Waits here for the loads of this set; no memory operation moves above.
  __device__ __forceinline__ void pin() const {
    q.pin();
    g.pin();
    pin_value(w);
    pin_value(mn);
  }
};

// v_mfma_f32_16x16x16 on four k values per lane (the path rows' k-steps).
template <typename E>
__device__ __forceinline__ f32x4 mfma16(s16x4 a, s16x4 b, f32x4 c) {
  if constexpr (__is_same(E, bf16)) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  } else {
    typedef __attribute__((ext_vector_type(4))) _Float16 h4;
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4, a), __builtin_bit_cast(h4, b), c, 0, 0, 0);
  }
}
template <typename E>
__device__ __forceinline__ s16x4 pack4(f32x4 x) {
  typedef __attribute__((ext_vector_type(4))) E e4;
  e4 v;
#pragma unroll
  for (int r = 0; r < 4; ++r) v[r] = (E)x[r];
  return __builtin_bit_cast(s16x4, v);
}

// gamma of one node's NB children in x[r0 .. r0 + NB) (logits in, gamma /
// scale out); depth d, the path's child jp, dl of the pair.
template <int NB>
__device__ __forceinline__ void path_gamma(f32x4& x, int r0, int d, int T, int jp, float dl, float maxhalf,
                                           float inv_scale) {
  if (d >= T) {
#pragma unroll
    for (int j = 0; j < NB; ++j) x[r0 + j] = 0.f;
    return;
  }
  float xc[NB], ev[NB];
  float mx = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    xc[j] = fminf(fmaxf(x[r0 + j], -maxhalf), maxhalf);
    mx = fmaxf(mx, xc[j]);
  }
  float se = 0.f;
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    ev[j] = __expf(xc[j] - mx);
    se += ev[j];
  }
  const float pa = dl / se;
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const float xv = x[r0 + j];
    const bool live = xv >= -maxhalf && xv <= maxhalf;
    x[r0 + j] = live ? ((j == jp ? dl : 0.f) - ev[j] * pa) * inv_scale : 0.f;
  }
}

template <typename E, int D, int LBP, int TR>
__global__ __launch_bounds__((64 * BwdTrTile<D, LBP, TR>::NW), (BwdTrTile<D, LBP, TR>::MINW)) void leaf_bwd_tr_kernel(
    LeafBwdArgs a) {
  static_assert(sizeof(E) == 2, "16-bit inputs");
  static_assert(TR % 16 == 0 && TR <= 32, "path rows: 0, 16 or 32");
  using M = Mfma<E>;
  using BT = BwdTrTile<D, LBP, TR>;
  constexpr int QT = BT::QT, RS = BT::RS, PS = BT::PS, ZS = BT::ZS;
  constexpr int NW = BT::NW;
  extern __shared__ __align__(16) char smem[];
  E* Ks = (E*)smem;        // [LBP][RS]
  E* Vs = Ks + LBP * RS;   // [LBP][RS]
  E* Qs = Vs + LBP * RS;   // [QT][RS]  Q rows of the tile
  E* Gs = Qs + QT * RS;    // [QT][RS]  dout rows of the tile
  E* Ps = Gs + QT * RS;    // [QT][PS]  w P rows
  E* Zs = Ps + QT * PS;    // [QT][ZS]  dz rows (keys, then path rows)
  E* Cs = Zs + QT * ZS;    // [TR][RS]  the path's child summaries

  int bh, beta;
  if (!xcd_bh_block(blockIdx.x, a.B * a.H, a.NL, bh, beta)) return;
  const int bb = bh / a.H, h = bh - bb * a.H;
  const int* bs = a.block_start + (int64_t)bh * (a.NL + 1);
  const int start = bs[beta], end = bs[beta + 1];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, col = lane & 15, g = lane >> 4;
  const int LB = a.LB, S = a.S;
  const int64_t LS = (int64_t)a.L * S;
  const E* q = (const E*)a.q;
  const E* k = (const E*)a.k;
  const E* v = (const E*)a.v;
  const E* go = (const E*)a.g;
  const int T = a.geo.T, lb = a.geo.lb, nrow = TR > 0 ? T * a.geo.b : 0;

  {  // stage the block's K and V rows: every load issued before the first LDS write
    constexpr int NST = (LBP * D / 8 + NW * 64 - 1) / (NW * 64);
    uint4 kr[NST], vr[NST];
#pragma unroll
    for (int i = 0; i < NST; ++i) {
      const int e = tid + i * NW * 64;
      const int key = e / (D / 8), c = (e - key * (D / 8)) * 8;
      const int64_t tok = (int64_t)beta * LB + key;
      const bool in = e < LBP * D / 8 && key < LB;
      kr[i] = in && k ? *(const uint4*)(k + bb * a.ksb + tok * a.ksl + h * a.ksh + c) : make_uint4(0, 0, 0, 0);
      vr[i] = in ? *(const uint4*)(v + bb * a.vsb + tok * a.vsl + h * a.vsh + c) : make_uint4(0, 0, 0, 0);
    }
    // path row e = d b + j: child j of the depth-d node over this block
    constexpr int NCS = TR > 0 ? (TR * D / 8 + NW * 64 - 1) / (NW * 64) : 1;
    uint4 cr[NCS];
    if constexpr (TR > 0) {
#pragma unroll
      for (int i = 0; i < NCS; ++i) {
        const int e = tid + i * NW * 64;
        const int row = e / (D / 8), c = (e - row * (D / 8)) * 8;
        cr[i] = make_uint4(0, 0, 0, 0);
        if (e < TR * D / 8 && row < nrow) {
          const int d = row >> lb, j = row & (a.geo.b - 1);
          const int srow = a.geo.off[d + 1] + ((beta >> (lb * (T - d))) << lb) + j;
          cr[i] = *(const uint4*)((const E*)a.sum_hi + ((int64_t)bh * a.NS + srow) * D + c);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < NST; ++i) {
      const int e = tid + i * NW * 64;
      const int key = e / (D / 8), c = (e - key * (D / 8)) * 8;
      if (e < LBP * D / 8) {
        *(uint4*)(Ks + key * RS + c) = kr[i];
        *(uint4*)(Vs + key * RS + c) = vr[i];
      }
    }
    if constexpr (TR > 0) {
#pragma unroll
      for (int i = 0; i < NCS; ++i) {
        const int e = tid + i * NW * 64;
        const int row = e / (D / 8), c = (e - row * (D / 8)) * 8;
        if (e < TR * D / 8) *(uint4*)(Cs + row * RS + c) = cr[i];
      }
    }
  }
  __syncthreads();

  // phase B: waves 0-3 accumulate dV = (wP)^T dout, waves 4-7 dK = dz^T Q;
  // wave w & 3 owns the quarter (key half (w & 3) >> 1, dim half w & 1):
  // MK2 x ND2 tiles of 16 x 16, MK2 + ND2 operand reads per MK2 * ND2 MFMAs
  constexpr int MK2 = LBP / 32, ND2 = D / 32;
  const bool dkw = w >= 4;
  const int mkb = MK2 * ((w & 3) >> 1), ndb = ND2 * (w & 1);
  const E* Ab = dkw ? Zs : Ps;
  const int AS = dkw ? ZS : PS;
  const E* Bb = dkw ? Qs : Gs;
  f32x4 acc[MK2][ND2];
#pragma unroll
  for (int x = 0; x < MK2; ++x)
#pragma unroll
    for (int y = 0; y < ND2; ++y) acc[x][y] = zero4();
  // path rows of dC = gamma^T Q: (TR / 16) x (D / 16) tiles, wave w takes w, w + NW, ...
  constexpr int NTE = (TR / 16) * (D / 16), NEW = (NTE + NW - 1) / NW;
  f32x4 cacc[NEW > 0 ? NEW : 1];
#pragma unroll
  for (int i = 0; i < (NEW > 0 ? NEW : 1); ++i) cacc[i] = zero4();

  // 128-key blocks (64-pair tiles): waves 0-3 run phase A of every tile and
  // waves 4-7 phase B, so phase B of a tile overlaps phase A of the next, and
  // no wave holds both the pair rows and the dV / dK accumulators.  Both
  // groups pass the same two barriers per tile: X (phase B of the previous
  // tile is done with the staging tiles) and Y (the tile is staged).
  constexpr bool kSplit = LBP > 64;
  static_assert(!kSplit || QT == 64, "split waves: 64-pair tiles");
  if constexpr (kSplit) {
    if (w >= 4) {
      const int c4 = w - 4;  // keys 32 c4 .. 32 c4 + 31, every head dim, dV and dK
      constexpr int NDT = D / 16, NEC = (NTE + 3) / 4;
      f32x4 av[2][NDT], ak[2][NDT], cc[NEC > 0 ? NEC : 1];
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < NDT; ++y) av[x][y] = ak[x][y] = zero4();
#pragma unroll
      for (int i = 0; i < (NEC > 0 ? NEC : 1); ++i) cc[i] = zero4();
      for (int t0 = start; t0 < end; t0 += QT) {
        __syncthreads();  // X
        __syncthreads();  // Y
#pragma unroll
        for (int ks = 0; ks < QT / M::K; ++ks) {
          const int ka = 32 * ks + 8 * g, kb = ka + 4;
          typename M::frag pv[2], zk[2];
#pragma unroll
          for (int x = 0; x < 2; ++x) {
            pv[x] = tr_frag(Ps, PS, ka, kb, 16 * (2 * c4 + x), lane);
            zk[x] = tr_frag(Zs, ZS, ka, kb, 16 * (2 * c4 + x), lane);
          }
#pragma unroll
          for (int y = 0; y < NDT; ++y) {
            const typename M::frag bg = tr_frag(Gs, RS, ka, kb, 16 * y, lane);
            const typename M::frag bq = tr_frag(Qs, RS, ka, kb, 16 * y, lane);
#pragma unroll
            for (int x = 0; x < 2; ++x) {
              av[x][y] = M::mma(pv[x], bg, av[x][y]);
              ak[x][y] = M::mma(zk[x], bq, ak[x][y]);
            }
          }
          if constexpr (TR > 0) {
#pragma unroll
            for (int i = 0; i < NEC; ++i) {
              const int t = c4 + 4 * i;
              if (NTE % 4 == 0 || t < NTE) {
                const int rt = t / NDT, dt = t - rt * NDT;
                cc[i] = M::mma(tr_frag(Zs, ZS, ka, kb, LBP + 16 * rt, lane), tr_frag(Qs, RS, ka, kb, 16 * dt, lane),
                               cc[i]);
              }
            }
          }
        }
      }
      if constexpr (TR > 0) {  // this block's path-row gradient (zero for a block without pairs)
        float* dc = a.dcp + ((int64_t)bh * a.NL + beta) * nrow * D;
#pragma unroll
        for (int i = 0; i < NEC; ++i) {
          const int t = c4 + 4 * i;
          if (NTE % 4 == 0 || t < NTE) {
            const int rt = t / NDT, dt = t - rt * NDT;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int e = 16 * rt + 4 * g + r;
              if (e < nrow) dc[(int64_t)e * D + 16 * dt + col] = cc[i][r] * a.scale;
            }
          }
        }
      }
      E* dv = (E*)a.dv;
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < NDT; ++y)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = 16 * (2 * c4 + x) + 4 * g + r;
            if (key < LB) {
              const int64_t tok = (int64_t)beta * LB + key;
              const int d = 16 * y + col;
              const int64_t th = (((int64_t)bb * a.N + tok) * a.H + h) * D + d;
              if (a.dk_leaf) acc1f(a.dk_leaf + th, ak[x][y][r] * a.scale, a.first);
              if (a.dv32) acc1f(a.dv32 + th, av[x][y][r], a.first);
              else dv[bb * a.vsb + tok * a.vsl + h * a.vsh + d] = (E)av[x][y][r];
            }
          }
      return;
    }
  }

  // Software pipeline over QT-pair tiles with two register sets: a tile
  // first waits for its own set (loaded one tile earlier), then issues the
  // loads of the next tile into the other set and reads the pair index of the
  // tile after.  The wait sits before the new loads on purpose: vmcnt counts
  // loads and stores alike, so any wait placed after them would also wait for
  // them.  The loop is unrolled twice so the sets never move between registers.
  const int* ord = a.order + (int64_t)bh * LS;
  const int pcol = 16 * w + col;  // this lane's pair column within the tile
  const bool aw = QT == 16 * NW || 16 * w < QT;  // the wave has pairs (phase A)
  auto idx = [&](int t) { return aw && t + pcol < end ? ord[t + pcol] : -1; };
  auto fetch = [&](int e, PairRows<E, D>& r) {  // pair entry e = l * S + u, or -1
    const int l = e >= 0 ? e / S : 0;
    r.l = e >= 0 ? l : -1;
    const int64_t qh = ((int64_t)bb * a.L + l) * a.H + h;
    r.sl = qh * S + (e >= 0 ? e - l * S : 0);
    r.q.load(e >= 0 ? q + bb * a.qsb + (int64_t)l * a.qsl + h * a.qsh : nullptr, g);
    r.g.load(e >= 0 ? go + bb * a.gsb + (int64_t)l * a.gsl + h * a.gsh : nullptr, g);
    r.w = e >= 0 ? a.slot_weight[r.sl] : 0.f;
    r.mn = TR > 0 && e >= 0 ? a.mean[qh] : 0.f;
  };
  auto tile = [&](const PairRows<E, D>& c) {
    const bool valid = c.l >= 0;
    const int l = valid ? c.l : 0;
    const int64_t sl = c.sl;
    const float wt = c.w;
    const RowFrags<E, D>& qc = c.q;
    const RowFrags<E, D>& gc = c.g;

    // ---- phase A: this wave's 16 pairs
    f32x4 sacc[LBP / 16], pacc[LBP / 16];
    f32x4 xacc[TR > 0 ? TR / 16 : 1];
    if (aw) {
#pragma unroll
    for (int mt = 0; mt < LBP / 16; ++mt) {
      sacc[mt] = zero4();
      pacc[mt] = zero4();
      const E* kp = Ks + (16 * mt + col) * RS + M::KPL * g;
      const E* vp = Vs + (16 * mt + col) * RS + M::KPL * g;
#pragma unroll
      for (int ks = 0; ks < D / M::K; ++ks) {
        sacc[mt] = M::mma(ld_frag(kp + ks * M::K), qc.f[ks], sacc[mt]);
        pacc[mt] = M::mma(ld_frag(vp + ks * M::K), gc.f[ks], pacc[mt]);
      }
    }
    if constexpr (TR > 0) {  // the path's child logits X = C_path Q^T
#pragma unroll
      for (int mt = 0; mt < TR / 16; ++mt) {
        xacc[mt] = zero4();
        const E* cp = Cs + (16 * mt + col) * RS + M::KPL * g;
#pragma unroll
        for (int ks = 0; ks < D / M::K; ++ks) xacc[mt] = M::mma(ld_frag(cp + ks * M::K), qc.f[ks], xacc[mt]);
      }
    }
    // keys < kmax are visible; masking only when some pair of the tile needs it
    const int kmax = valid ? (a.causal ? min(LB, l + (a.N - a.L) - beta * LB + 1) : LB) : 0;
    if (__any(kmax < LBP)) {
#pragma unroll
      for (int mt = 0; mt < LBP / 16; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          sacc[mt][r] = (16 * mt + 4 * g + r) < kmax ? sacc[mt][r] * a.scale_log2 : -__builtin_inff();
    } else {
#pragma unroll
      for (int mt = 0; mt < LBP / 16; ++mt) sacc[mt] *= a.scale_log2;
    }
    float mx = -__builtin_inff();
#pragma unroll
    for (int mt = 0; mt < LBP / 16; ++mt)
      mx = fmaxf(mx, fmaxf(fmaxf(sacc[mt][0], sacc[mt][1]), fmaxf(sacc[mt][2], sacc[mt][3])));
    mx = col_max(mx);
    if (mx == -__builtin_inff()) mx = 0.f;  // no visible key (padding pairs): all p = 0
    float sum = 0.f;
#pragma unroll
    for (int mt = 0; mt < LBP / 16; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pv = __builtin_amdgcn_exp2f(sacc[mt][r] - mx);
        sacc[mt][r] = pv;
        sum += pv;
      }
    sum = col_sum(sum);
    const float inv = sum > 0.f ? __builtin_amdgcn_rcpf(sum) : 0.f;
    float delta = 0.f;
#pragma unroll
    for (int mt = 0; mt < LBP / 16; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sacc[mt][r] *= inv;
        delta += sacc[mt][r] * pacc[mt][r];
      }
    delta = col_sum(delta);
#pragma unroll
    for (int mt = 0; mt < LBP / 16; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) pacc[mt][r] = wt * sacc[mt][r] * (pacc[mt][r] - delta);
    if constexpr (TR == 0) {
      if (valid && g == 0) a.delta[sl] = delta;
    } else {
      // the path rows' gamma / scale (scaled back by the products' scale);
      // rows 16 mt + 4 g + r: b = 4 one node's children, b = 2 two nodes'
      const float dl = wt * (delta - c.mn);  // padding pairs: wt = 0
#pragma unroll
      for (int mt = 0; mt < TR / 16; ++mt) {
        if (lb == 2) {
          const int d = 4 * mt + g;
          const int jp = d < T ? (beta >> (2 * (T - 1 - d))) & 3 : 0;
          path_gamma<4>(xacc[mt], 0, d, T, jp, dl, a.maxhalf, a.inv_scale);
        } else {
          const int d = 8 * mt + 2 * g;
          const int jp0 = d < T ? (beta >> (T - 1 - d)) & 1 : 0;
          const int jp1 = d + 1 < T ? (beta >> (T - 2 - d)) & 1 : 0;
          path_gamma<2>(xacc[mt], 0, d, T, jp0, dl, a.maxhalf, a.inv_scale);
          path_gamma<2>(xacc[mt], 2, d + 1, T, jp1, dl, a.maxhalf, a.inv_scale);
        }
      }
    }

    // dq_pair^T = K^T dz^T: K^T fragments read transposed from Ks in the
    // accumulator's key order (keys 32ks + 4g.. and 32ks + 16 + 4g..)
    // K^T fragments with permuted head dims: each lane ends with eight
    // consecutive dims of its pair's dq row, one 16-byte store per 32 dims;
    // the path rows add C_path^T gamma^T, four rows per k-step
    E* dqp = (E*)a.dq_part + sl * D + 8 * g;
#pragma unroll
    for (int p = 0; p < D / 32; ++p) {
      f32x4 o0 = zero4(), o1 = zero4();
#pragma unroll
      for (int ks = 0; ks < LBP / M::K; ++ks) {
        const typename M::frag z = acc_operand<E>(pacc, ks);
        o0 = M::mma(perm_dim_frag<E>(Ks, RS, 2 * p, ks, lane), z, o0);
        o1 = M::mma(perm_dim_frag<E>(Ks, RS, 2 * p + 1, ks, lane), z, o1);
      }
      if constexpr (TR > 0) {
        const int cc = 32 * p + 8 * (col & 3);
#pragma unroll
        for (int mt = 0; mt < TR / 16; ++mt) {
          const s16x4 z = pack4<E>(xacc[mt]);
          const int row = 16 * mt + 4 * g + (col >> 2);
          o0 = mfma16<E>(tr_read4(Cs, RS, row, cc), z, o0);
          o1 = mfma16<E>(tr_read4(Cs, RS, row, cc + 4), z, o1);
        }
      }
      if (valid) {
        typedef __attribute__((ext_vector_type(8))) E e8;
        e8 o;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          o[r] = (E)(o0[r] * a.scale);
          o[4 + r] = (E)(o1[r] * a.scale);
        }
        *(e8*)(dqp + 32 * p) = o;
      }
    }

    }  // aw

    __syncthreads();  // phase B of the previous tile is done with the staging tiles
    if (aw) {
      E* pr = Ps + pcol * PS + 4 * g;
      E* zr = Zs + pcol * ZS + 4 * g;
#pragma unroll
      for (int mt = 0; mt < LBP / 16; ++mt) {
        typedef __attribute__((ext_vector_type(4))) E e4;
        e4 pv, zv;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          pv[r] = (E)(wt * sacc[mt][r]);
          zv[r] = (E)pacc[mt][r];
        }
        *(e4*)(pr + 16 * mt) = pv;
        *(e4*)(zr + 16 * mt) = zv;
      }
      if constexpr (TR > 0) {
#pragma unroll
        for (int mt = 0; mt < TR / 16; ++mt) *(s16x4*)(zr + LBP + 16 * mt) = pack4<E>(xacc[mt]);
      }
#pragma unroll
      for (int ks = 0; ks < D / M::K; ++ks) {
        *(typename M::frag*)(Qs + pcol * RS + ks * M::K + M::KPL * g) = qc.f[ks];
        *(typename M::frag*)(Gs + pcol * RS + ks * M::K + M::KPL * g) = gc.f[ks];
      }
    }
    __syncthreads();

    // ---- phase B: this wave's block of dV or dK over the tile's pairs, and
    // its tiles of the path rows' dC (split waves: waves 4-7, above)
    if constexpr (!kSplit) {
#pragma unroll
    for (int ks = 0; ks < QT / M::K; ++ks) {
      const int ka = 32 * ks + 8 * g, kb = ka + 4;
      typename M::frag af[MK2], bf[ND2];
#pragma unroll
      for (int x = 0; x < MK2; ++x) af[x] = tr_frag(Ab, AS, ka, kb, 16 * (mkb + x), lane);
#pragma unroll
      for (int y = 0; y < ND2; ++y) bf[y] = tr_frag(Bb, RS, ka, kb, 16 * (ndb + y), lane);
#pragma unroll
      for (int x = 0; x < MK2; ++x)
#pragma unroll
        for (int y = 0; y < ND2; ++y) acc[x][y] = M::mma(af[x], bf[y], acc[x][y]);
      if constexpr (TR > 0) {
#pragma unroll
        for (int i = 0; i < NEW; ++i) {
          const int t = w + NW * i;
          if (NTE % NW == 0 || t < NTE) {
            const int rt = t / (D / 16), dt = t - rt * (D / 16);
            cacc[i] = M::mma(tr_frag(Zs, ZS, ka, kb, LBP + 16 * rt, lane), tr_frag(Qs, RS, ka, kb, 16 * dt, lane),
                             cacc[i]);
          }
        }
      }
    }
    }  // !kSplit
  };

  PairRows<E, D> ra, rb;
  int e1 = idx(start + QT);
  fetch(idx(start), ra);
  for (int t0 = start; t0 < end; t0 += 2 * QT) {
    ra.pin();
    const int e2 = idx(t0 + 2 * QT);
    fetch(e1, rb);
    tile(ra);
    if (t0 + QT >= end) break;
    rb.pin();
    e1 = idx(t0 + 3 * QT);
    fetch(e2, ra);
    tile(rb);
  }
  if constexpr (kSplit) return;  // waves 4-7 write the block's gradients

  if constexpr (TR > 0) {  // this block's path-row gradient (zero for a block without pairs)
    float* dc = a.dcp + ((int64_t)bh * a.NL + beta) * nrow * D;
#pragma unroll
    for (int i = 0; i < NEW; ++i) {
      const int t = w + NW * i;
      if (NTE % NW == 0 || t < NTE) {
        const int rt = t / (D / 16), dt = t - rt * (D / 16);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int e = 16 * rt + 4 * g + r;
          if (e < nrow) dc[(int64_t)e * D + 16 * dt + col] = cacc[i][r] * a.scale;
        }
      }
    }
  }

  E* dv = (E*)a.dv;
  if (dkw && !a.dk_leaf) return;
#pragma unroll
  for (int x = 0; x < MK2; ++x)
#pragma unroll
    for (int y = 0; y < ND2; ++y)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = 16 * (mkb + x) + 4 * g + r;
        if (key < LB) {
          const int64_t tok = (int64_t)beta * LB + key;
          const int d = 16 * (ndb + y) + col;
          const int64_t th = (((int64_t)bb * a.N + tok) * a.H + h) * D + d;
          if (dkw) acc1f(a.dk_leaf + th, acc[x][y][r] * a.scale, a.first);
          else if (a.dv32) acc1f(a.dv32 + th, acc[x][y][r], a.first);
          else dv[bb * a.vsb + tok * a.vsl + h * a.vsh + d] = (E)acc[x][y][r];
        }
      }
}

// Launches leaf_bwd_tr_kernel<E, D, LBP, TR> with the arguments of a.
template <typename E, int D, int LBP, int TR>
hipError_t launch_bwd_tr(const LeafBwdArgs& a, unsigned grid, hipStream_t st) {
  constexpr int smem = BwdTrTile<D, LBP, TR>::bytes;
  static_assert(smem <= 160 * 1024, "the tile must fit the LDS");
  hipError_t e = hipFuncSetAttribute((const void*)leaf_bwd_tr_kernel<E, D, LBP, TR>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, smem);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((leaf_bwd_tr_kernel<E, D, LBP, TR>), dim3(grid), dim3(64 * BwdTrTile<D, LBP, TR>::NW), smem, st,
                     a);
  return hipGetLastError();
}

// leaf_bwd_path.hip: the TR = 16 / 32 variants (P.path_rows), dispatched on
// dtype, head dim and padded block size.
hipError_t launch_leaf_bwd_path(const Plan& P, const LeafBwdArgs& a, unsigned grid, hipStream_t st);

}  // namespace ta
