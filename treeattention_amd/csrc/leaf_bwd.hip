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
#include "leaf_bwd_tr.h"

namespace ta {


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


template <typename E, int D, int LBP>
static int bwd_smem_t() {
  return BwdTile<D, LBP, (int)sizeof(E)>::bytes;
}

int leaf_bwd_smem(const Plan& P) {
  const int D = (int)P.D, LBP = padded_keys(P.geo.LB), ES = P.esize;
  if (ES == 2) {  // the transposing-read kernel (BwdTrTile), with the plan's path rows
    const int TR = P.path_rows;
    const int s = bwd_tr_bytes(D, LBP, TR, bwd_tr_qt(D, LBP, TR));
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
  if (P.path_rows) {
    // the tree gradient along every pair's path (the plan allows it only for
    // 16-bit inputs whose tile with the path rows fits the LDS)
    a.delta = nullptr;
    a.geo = P.geo;
    a.NS = P.geo.NS;
    a.maxhalf = 0.5f * P.p.max_logit;
    a.inv_scale = 1.f / P.p.scale;
    a.sum_hi = rec + P.rec.sum_hi;
    a.dcp = (float*)(ws + P.bws.dcp);
    if (P.acc.mean) {
      a.mean = P.acc.mean;  // a chunk: dout . out over all samples, computed once
    } else {
      float* mean = (float*)(ws + P.bws.mean);
      hipError_t e = launch_chunk_mean(P, g, rec + P.rec.out_e, true, mean, st);
      if (e != hipSuccess) return e;
      a.mean = mean;
    }
    return launch_leaf_bwd_path(P, a, grid, st);
  }
  constexpr int smem8 = BwdTrTile<D, LBP, 0>::bytes;
  if constexpr (sizeof(E) == 2 && LBP >= 32 && smem8 <= 160 * 1024) {
    return launch_bwd_tr<E, D, LBP, 0>(a, grid, st);
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
