// K4a: leaf-block backward.
//
// One workgroup per (leaf block, batch*head) walks every (query, leaf block)
// pair of its bucket in 64-pair tiles and keeps dV_blk and dK_blk in
// registers for the whole bucket, so each leaf token's gradient is produced
// by exactly one workgroup in a fixed order: no atomics (the reference
// scatters with gpuAtomicAdd, scatter_weighted_grad_v.cu:49-52 and
// accumulate_qk_non_causal.cu:71-74).  Per tile (g = output gradient row of
// the pair's query, w = the pair's summed sample weight):
//   S^T = K Q^T, P = softmax over keys             (recomputed)
//   dP^T = V g^T, delta = sum_keys P dP = g . o     (-> the tree backward)
//   dz = w P (dP - delta)
//   dq_pair^T = scale K^T dz^T                     (-> per-pair slot, summed in tree_bwd)
//   dV += (w P)^T g,  dK += scale dz^T Q            (P^T and dz^T staged in LDS)
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
  float* delta;     // (B,L,H,S)
  void* dq_part;    // E (B,L,H,S,D)
  void* dv;         // E, v strides
  float* dk_leaf;   // (B,N,H,D) or null
  float* dv32;      // chunked problem: dv as float (B,N,H,D) rows, else null
  int first;        // chunked problem: the first chunk writes dv32 / dk_leaf, later ones add
};

// One element of the float accumulators of a chunked problem (or of dk_leaf).
__device__ __forceinline__ void acc1f(float* p, float x, int first) { *p = first ? x : *p + x; }

template <typename E>
__device__ __forceinline__ void mov8(E* o, const E* p) {
  if constexpr (sizeof(E) == 2) {
    *(uint4*)o = *(const uint4*)p;
  } else {
    *(float4*)o = *(const float4*)p;
    *(float4*)(o + 4) = *(const float4*)(p + 4);
  }
}
template <typename E>
__device__ __forceinline__ void zero8e(E* o) {
  if constexpr (sizeof(E) == 2) {
    *(uint4*)o = make_uint4(0, 0, 0, 0);
  } else {
    *(float4*)o = make_float4(0, 0, 0, 0);
    *(float4*)(o + 4) = make_float4(0, 0, 0, 0);
  }
}

// Pair tiles of QT = 64 pairs (16 per wave in phase A) with K^T kept in LDS
// for the dq product when it fits; where the K / V block, the tile's rows and
// its (wP)^T, dz^T tiles would exceed the 160 KiB of LDS (float inputs with
// large head dims or blocks) the tile shrinks to 32 or 16 pairs, phase A on
// the first QT / 16 waves, and K^T is read from the K rows instead.
// When even 16-pair tiles do not fit (float, head dim 128, 128-key blocks),
// V stays in global memory (L2-resident, 64 KB per block) and phase A reads
// its MFMA operands from there: 32-pair tiles.
template <int D, int LBP, int ES>
struct BwdTile {
  static constexpr int RS = D + 8, TS = LBP + 8;  // padded LDS row strides
  static constexpr int bytes_for(int qt, bool kt, bool vs) {
    return ((vs ? 2 : 1) * LBP * RS + 2 * qt * RS + 2 * LBP * (qt + 8) + (kt ? D * TS : 0)) * ES + 64 * 4;
  }
  static constexpr bool kKt64 = (LBP <= 64) || ES == 2 && D <= 64;
  static constexpr int kMax = 160 * 1024;
  static constexpr bool kVg = bytes_for(16, false, true) > kMax;  // V read from global memory
  static constexpr int QT = kVg ? 32
                            : bytes_for(64, kKt64, true) <= kMax ? 64
                            : bytes_for(32, false, true) <= kMax ? 32 : 16;
  static constexpr bool kKt = QT == 64 && kKt64 && !kVg;
  static constexpr int PS = QT + 8;
  static constexpr int bytes = bytes_for(QT, kKt, !kVg);
};

template <typename E, int D, int LBP>
__global__ __launch_bounds__(256) void leaf_bwd_kernel(LeafBwdArgs a) {
  using M = Mfma<E>;
  using BT = BwdTile<D, LBP, (int)sizeof(E)>;
  constexpr int QT = BT::QT, RS = BT::RS, PS = BT::PS, TS = BT::TS;
  constexpr int NT = (LBP / 16) * (D / 16) / 4;  // dV / dK tiles per wave
  extern __shared__ __align__(16) char smem[];
  E* Ks = (E*)smem;        // [LBP][RS]
  E* Vs = Ks + LBP * RS;   // [LBP][RS] (unless kVg)
  E* Qs = Vs + (BT::kVg ? 0 : LBP * RS);  // [QT][RS]
  E* Gs = Qs + QT * RS;    // [QT][RS]
  E* Pt = Gs + QT * RS;    // [LBP][PS]  (w P)^T
  E* Zt = Pt + LBP * PS;   // [LBP][PS]  dz^T
  E* Kt = Zt + LBP * PS;   // [D][TS]    K^T (if kKt)
  int* ent_s = (int*)(Kt + (BT::kKt ? D * TS : 0));

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

  for (int e = tid; e < LBP * D / 8; e += 256) {
    const int key = e / (D / 8), c = (e - key * (D / 8)) * 8;
    const int64_t tok = (int64_t)beta * LB + key;
    if (key < LB && k) mov8(Ks + key * RS + c, k + bb * a.ksb + tok * a.ksl + h * a.ksh + c);
    else zero8e(Ks + key * RS + c);
    if constexpr (!BT::kVg) {
      if (key < LB) mov8(Vs + key * RS + c, v + bb * a.vsb + tok * a.vsl + h * a.vsh + c);
      else zero8e(Vs + key * RS + c);
    }
    if constexpr (BT::kKt) {
#pragma unroll
      for (int i = 0; i < 8; ++i) Kt[(c + i) * TS + key] = Ks[key * RS + c + i];
    }
  }

  f32x4 dvacc[NT], dkacc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) { dvacc[t] = zero4(); dkacc[t] = zero4(); }

  for (int t0 = start; t0 < end; t0 += QT) {
    __syncthreads();
    if (tid < QT) ent_s[tid] = (t0 + tid < end) ? a.order[(int64_t)bh * LS + t0 + tid] : -1;
    __syncthreads();
    for (int e = tid; e < QT * D / 8; e += 256) {
      const int r = e / (D / 8), c = (e - r * (D / 8)) * 8;
      const int ent = ent_s[r];
      if (ent >= 0) {
        const int l = ent / S;
        mov8(Qs + r * RS + c, q + bb * a.qsb + (int64_t)l * a.qsl + h * a.qsh + c);
        mov8(Gs + r * RS + c, go + bb * a.gsb + (int64_t)l * a.gsl + h * a.gsh + c);
      } else {
        zero8e(Qs + r * RS + c);
        zero8e(Gs + r * RS + c);
      }
    }
    __syncthreads();

    if (16 * w < QT) {  // phase A: this wave's 16 pairs of the tile
    const int qcol = 16 * w + col;
    const int ent = ent_s[qcol];
    const bool valid = ent >= 0;
    const int l = valid ? ent / S : 0, u = valid ? ent - l * S : 0;
    const int64_t qh = ((int64_t)bb * a.L + l) * a.H + h;

    f32x4 sacc[LBP / 16], pacc[LBP / 16];
#pragma unroll
    for (int mt = 0; mt < LBP / 16; ++mt) {
      sacc[mt] = zero4();
      pacc[mt] = zero4();
      const E* kp = Ks + (16 * mt + col) * RS + M::KPL * g;
      const E* qp = Qs + qcol * RS + M::KPL * g;
      const E* gp = Gs + qcol * RS + M::KPL * g;
      if constexpr (BT::kVg) {
        // V rows from global memory (keys past LB are zero)
        const int key = 16 * mt + col;
        const E* vg = v + bb * a.vsb + ((int64_t)beta * LB + (key < LB ? key : 0)) * a.vsl + h * a.vsh + M::KPL * g;
        const bool kin = key < LB;
#pragma unroll
        for (int ks = 0; ks < D / M::K; ++ks) {
          sacc[mt] = M::mma(ld_frag(kp + ks * M::K), ld_frag(qp + ks * M::K), sacc[mt]);
          const E vv = kin ? vg[ks * M::K] : (E)0.f;
          pacc[mt] = M::mma(vv, ld_frag(gp + ks * M::K), pacc[mt]);
        }
      } else {
        const E* vp = Vs + (16 * mt + col) * RS + M::KPL * g;
#pragma unroll
        for (int ks = 0; ks < D / M::K; ++ks) {
          sacc[mt] = M::mma(ld_frag(kp + ks * M::K), ld_frag(qp + ks * M::K), sacc[mt]);
          pacc[mt] = M::mma(ld_frag(vp + ks * M::K), ld_frag(gp + ks * M::K), pacc[mt]);
        }
      }
    }
    const int kmax = valid ? (a.causal ? min(LB, l + (a.N - a.L) - beta * LB + 1) : LB) : 0;
    float mx = -__builtin_inff();
#pragma unroll
    for (int mt = 0; mt < LBP / 16; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float s = (16 * mt + 4 * g + r) < kmax ? sacc[mt][r] * a.scale_log2 : -__builtin_inff();
        sacc[mt][r] = s;
        mx = fmaxf(mx, s);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    float sum = 0.f;
#pragma unroll
    for (int mt = 0; mt < LBP / 16; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = (16 * mt + 4 * g + r) < kmax ? exp2f(sacc[mt][r] - mx) : 0.f;
        sacc[mt][r] = p;
        sum += p;
      }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    const float inv = sum > 0.f ? 1.f / sum : 0.f;
    float delta = 0.f;
#pragma unroll
    for (int mt = 0; mt < LBP / 16; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sacc[mt][r] *= inv;
        delta += sacc[mt][r] * pacc[mt][r];
      }
    delta += __shfl_xor(delta, 16, 64);
    delta += __shfl_xor(delta, 32, 64);
    const float wt = valid ? a.slot_weight[qh * S + u] : 0.f;
#pragma unroll
    for (int mt = 0; mt < LBP / 16; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = 16 * mt + 4 * g + r;
        const float p = sacc[mt][r];
        const float dz = wt * p * (pacc[mt][r] - delta);
        pacc[mt][r] = dz;
        Pt[key * PS + qcol] = (E)(wt * p);
        Zt[key * PS + qcol] = (E)dz;
      }
    if (valid && g == 0) a.delta[qh * S + u] = delta;

    E* dqp = (E*)a.dq_part + (qh * S + u) * D;
#pragma unroll
    for (int md = 0; md < D / 16; ++md) {
      f32x4 o = zero4();
#pragma unroll
      for (int ks = 0; ks < LBP / M::K; ++ks) {
        if constexpr (BT::kKt)
          o = M::mma(ld_frag_perm(Kt + (16 * md + col) * TS, ks, g), acc_operand<E>(pacc, ks), o);
        else
          o = M::mma(ld_frag_perm_strided<E>(Ks + 16 * md + col, RS, ks, g), acc_operand<E>(pacc, ks), o);
      }
      if (valid) store4(dqp + 16 * md + 4 * g, o, a.scale);
    }
    }
    __syncthreads();

#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int tile = w + 4 * t;
      const int mk = tile / (D / 16), nd = tile - mk * (D / 16);
      const E* pa = Pt + (16 * mk + col) * PS + M::KPL * g;
      const E* za = Zt + (16 * mk + col) * PS + M::KPL * g;
      const E* gb = Gs + (M::KPL * g) * RS + 16 * nd + col;
      const E* qb = Qs + (M::KPL * g) * RS + 16 * nd + col;
#pragma unroll
      for (int ks = 0; ks < QT / M::K; ++ks) {
        dvacc[t] = M::mma(ld_frag(pa + ks * M::K), ld_frag_strided(gb + ks * M::K * RS, RS), dvacc[t]);
        dkacc[t] = M::mma(ld_frag(za + ks * M::K), ld_frag_strided(qb + ks * M::K * RS, RS), dkacc[t]);
      }
    }
  }

  E* dv = (E*)a.dv;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int tile = w + 4 * t;
    const int mk = tile / (D / 16), nd = tile - mk * (D / 16);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = 16 * mk + 4 * g + r;
      if (key < LB) {
        const int64_t tok = (int64_t)beta * LB + key;
        const int d = 16 * nd + col;
        const int64_t th = (((int64_t)bb * a.N + tok) * a.H + h) * D + d;
        if (a.dv32) acc1f(a.dv32 + th, dvacc[t][r], a.first);
        else dv[bb * a.vsb + tok * a.vsl + h * a.vsh + d] = (E)dvacc[t][r];
        if (a.dk_leaf) acc1f(a.dk_leaf + th, dkacc[t][r] * a.scale, a.first);
      }
    }
  }
}

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
// per wave; 128-key blocks take 64-pair tiles (so the K / V, pair-row and
// P / dz tiles fit the LDS), whose phase A runs on waves 0-3 while all eight
// share phase B.
template <int D, int LBP>
struct BwdTrTile {
  static constexpr int NW = 8;                      // waves
  static constexpr int QT = LBP > 64 ? 64 : 128;    // pairs per tile, 16 per phase-A wave
  static constexpr int RS = D + 16, PS = LBP + 16;
  static constexpr int bytes = (2 * LBP * RS + 2 * QT * RS + 2 * QT * PS) * 2;
};


// One pair column's operands for a tile: query and output-gradient row
// fragments, the pair's summed sample weight, its query row (-1: padding) and
// its (b, l, h, u) slot.
template <typename E, int D>
struct PairRows {
  RowFrags<E, D> q, g;
  float w;
  int l;
  int64_t sl;
  // Waits here for the loads of this set; no memory operation moves above.
  __device__ __forceinline__ void pin() const {
    q.pin();
    g.pin();
    pin_value(w);
  }
};

template <typename E, int D, int LBP>
__global__ __launch_bounds__((64 * BwdTrTile<D, LBP>::NW)) void leaf_bwd_tr_kernel(LeafBwdArgs a) {
  static_assert(sizeof(E) == 2, "16-bit inputs");
  using M = Mfma<E>;
  using BT = BwdTrTile<D, LBP>;
  constexpr int QT = BT::QT, RS = BT::RS, PS = BT::PS;
  constexpr int NW = BT::NW;
  extern __shared__ __align__(16) char smem[];
  E* Ks = (E*)smem;        // [LBP][RS]
  E* Vs = Ks + LBP * RS;   // [LBP][RS]
  E* Qs = Vs + LBP * RS;   // [QT][RS]  Q rows of the tile
  E* Gs = Qs + QT * RS;    // [QT][RS]  dout rows of the tile
  E* Ps = Gs + QT * RS;    // [QT][PS]  w P rows
  E* Zs = Ps + QT * PS;    // [QT][PS]  dz rows

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
#pragma unroll
    for (int i = 0; i < NST; ++i) {
      const int e = tid + i * NW * 64;
      const int key = e / (D / 8), c = (e - key * (D / 8)) * 8;
      if (e < LBP * D / 8) {
        *(uint4*)(Ks + key * RS + c) = kr[i];
        *(uint4*)(Vs + key * RS + c) = vr[i];
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
  const E* Bb = dkw ? Qs : Gs;
  f32x4 acc[MK2][ND2];
#pragma unroll
  for (int x = 0; x < MK2; ++x)
#pragma unroll
    for (int y = 0; y < ND2; ++y) acc[x][y] = zero4();

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
    r.sl = (((int64_t)bb * a.L + l) * a.H + h) * S + (e >= 0 ? e - l * S : 0);
    r.q.load(e >= 0 ? q + bb * a.qsb + (int64_t)l * a.qsl + h * a.qsh : nullptr, g);
    r.g.load(e >= 0 ? go + bb * a.gsb + (int64_t)l * a.gsl + h * a.gsh : nullptr, g);
    r.w = e >= 0 ? a.slot_weight[r.sl] : 0.f;
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
    if (valid && g == 0) a.delta[sl] = delta;

    // dq_pair^T = K^T dz^T: K^T fragments read transposed from Ks in the
    // accumulator's key order (keys 32ks + 4g.. and 32ks + 16 + 4g..)
    // K^T fragments with permuted head dims: each lane ends with eight
    // consecutive dims of its pair's dq row, one 16-byte store per 32 dims
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
      E* zr = Zs + pcol * PS + 4 * g;
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
#pragma unroll
      for (int ks = 0; ks < D / M::K; ++ks) {
        *(typename M::frag*)(Qs + pcol * RS + ks * M::K + M::KPL * g) = qc.f[ks];
        *(typename M::frag*)(Gs + pcol * RS + ks * M::K + M::KPL * g) = gc.f[ks];
      }
    }
    __syncthreads();

    // ---- phase B: this wave's block of dV or dK over the tile's pairs
#pragma unroll
    for (int ks = 0; ks < QT / M::K; ++ks) {
      const int ka = 32 * ks + 8 * g, kb = ka + 4;
      typename M::frag af[MK2], bf[ND2];
#pragma unroll
      for (int x = 0; x < MK2; ++x) af[x] = tr_frag(Ab, PS, ka, kb, 16 * (mkb + x), lane);
#pragma unroll
      for (int y = 0; y < ND2; ++y) bf[y] = tr_frag(Bb, RS, ka, kb, 16 * (ndb + y), lane);
#pragma unroll
      for (int x = 0; x < MK2; ++x)
#pragma unroll
        for (int y = 0; y < ND2; ++y) acc[x][y] = M::mma(af[x], bf[y], acc[x][y]);
    }
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

template <typename E, int D, int LBP>
static int bwd_smem_t() {
  return BwdTile<D, LBP, (int)sizeof(E)>::bytes;
}

int leaf_bwd_smem(const Plan& P) {
  const int D = (int)P.D, LBP = padded_keys(P.geo.LB), ES = P.esize;
  if (ES == 2) {  // the transposing-read kernel (BwdTrTile)
    const int QT = LBP > 64 ? 64 : 128, RS = D + 16, PS = LBP + 16;
    const int s = (2 * LBP * RS + 2 * QT * RS + 2 * QT * PS) * 2;
    return s <= 160 * 1024 ? s : -1;
  }
  int s = 0;
  switch (D * 1000 + LBP) {
#define TA_BWD_TILE(d, lbp) \
  case d * 1000 + lbp: s = ES == 2 ? BwdTile<d, lbp, 2>::bytes : BwdTile<d, lbp, 4>::bytes; break;
    TA_BWD_TILE(32, 32) TA_BWD_TILE(32, 64) TA_BWD_TILE(32, 128)
    TA_BWD_TILE(64, 32) TA_BWD_TILE(64, 64) TA_BWD_TILE(64, 128)
    TA_BWD_TILE(96, 32) TA_BWD_TILE(96, 64) TA_BWD_TILE(96, 128)
    TA_BWD_TILE(128, 32) TA_BWD_TILE(128, 64) TA_BWD_TILE(128, 128)
#undef TA_BWD_TILE
    default: return -1;
  }
  return s <= 160 * 1024 ? s : -1;
}

template <typename E, int D, int LBP>
static hipError_t leaf_bwd_impl(const Plan& P, const void* q, const void* k, const void* v, const void* g,
                                const char* rec, void* dv, char* ws, hipStream_t st) {
  LeafBwdArgs a;
  a.B = (int)P.B;
  a.L = (int)P.L;
  a.N = (int)P.N;
  a.H = (int)P.H;
  a.S = (int)P.S;
  a.NL = P.geo.NL;
  a.LB = P.geo.LB;
  a.causal = P.p.causal == TA_CAUSAL_EXACT;
  a.scale = P.p.scale;
  a.scale_log2 = P.p.scale * 1.4426950408889634f;
  const bool nodekeys = P.p.tree_mode == TA_TREE_NODEKEYS;
  a.q = q;
  a.k = nodekeys ? nullptr : k;
  a.v = v;
  a.g = g;
  a.qsb = P.p.q_strides[0]; a.qsl = P.p.q_strides[1]; a.qsh = P.p.q_strides[2];
  a.ksb = P.p.k_strides[0]; a.ksl = P.p.k_strides[1]; a.ksh = P.p.k_strides[2];
  a.vsb = P.p.v_strides[0]; a.vsl = P.p.v_strides[1]; a.vsh = P.p.v_strides[2];
  a.gsb = P.p.g_strides[0]; a.gsl = P.p.g_strides[1]; a.gsh = P.p.g_strides[2];
  a.order = (const int*)(rec + P.rec.order);
  a.block_start = (const int*)(rec + P.rec.block_start);
  a.slot_weight = (const float*)(rec + P.rec.slot_weight);
  a.delta = (float*)(ws + P.bws.delta);
  a.dq_part = ws + P.bws.dq_part;
  a.dv = dv;
  a.dk_leaf = nodekeys ? nullptr : P.acc.dk_leaf ? P.acc.dk_leaf : (float*)(ws + P.bws.dk_leaf);
  a.dv32 = P.acc.dv32;
  a.first = P.acc.dv32 ? P.acc.first : 1;  // one launch: plain writes
  const unsigned grid = xcd_grid(P.BH, P.geo.NL);
  constexpr int smem8 = BwdTrTile<D, LBP>::bytes;
  if constexpr (sizeof(E) == 2 && LBP >= 32 && smem8 <= 160 * 1024) {
    hipError_t e = hipFuncSetAttribute((const void*)leaf_bwd_tr_kernel<E, D, LBP>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, smem8);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((leaf_bwd_tr_kernel<E, D, LBP>), dim3(grid), dim3(64 * BwdTrTile<D, LBP>::NW), smem8, st, a);
  } else {
    const int smem = bwd_smem_t<E, D, LBP>();
    hipError_t e = hipFuncSetAttribute((const void*)leaf_bwd_kernel<E, D, LBP>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, smem);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((leaf_bwd_kernel<E, D, LBP>), dim3(grid), dim3(256), smem, st, a);
  }
  return hipGetLastError();
}

template <typename E, int D>
static hipError_t leaf_bwd_lb(const Plan& P, const void* q, const void* k, const void* v, const void* g,
                              const char* rec, void* dv, char* ws, hipStream_t st) {
  switch (padded_keys(P.geo.LB)) {
    case 32: return leaf_bwd_impl<E, D, 32>(P, q, k, v, g, rec, dv, ws, st);
    case 64: return leaf_bwd_impl<E, D, 64>(P, q, k, v, g, rec, dv, ws, st);
    default: return leaf_bwd_impl<E, D, 128>(P, q, k, v, g, rec, dv, ws, st);
  }
}

template <typename E>
static hipError_t leaf_bwd_d(const Plan& P, const void* q, const void* k, const void* v, const void* g,
                             const char* rec, void* dv, char* ws, hipStream_t st) {
  switch (P.D) {
    case 32: return leaf_bwd_lb<E, 32>(P, q, k, v, g, rec, dv, ws, st);
    case 64: return leaf_bwd_lb<E, 64>(P, q, k, v, g, rec, dv, ws, st);
    case 96: return leaf_bwd_lb<E, 96>(P, q, k, v, g, rec, dv, ws, st);
    default: return leaf_bwd_lb<E, 128>(P, q, k, v, g, rec, dv, ws, st);
  }
}

hipError_t launch_leaf_bwd(const Plan& P, const void* q, const void* k, const void* v, const void* g,
                           const char* rec, void* dv, char* ws, hipStream_t st) {
  if (P.geo.LB == 1) return launch_gather_bwd(P, v, g, dv, rec, ws, st);
  switch (P.p.dtype) {
    case TA_F32: return leaf_bwd_d<float>(P, q, k, v, g, rec, dv, ws, st);
    case TA_BF16: return leaf_bwd_d<bf16>(P, q, k, v, g, rec, dv, ws, st);
    default: return leaf_bwd_d<f16>(P, q, k, v, g, rec, dv, ws, st);
  }
}

}  // namespace ta
