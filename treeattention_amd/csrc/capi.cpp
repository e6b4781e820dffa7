// C ABI of the tree-attention library: validation, buffer layouts, launch order.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <string>

#include "launch.h"

namespace ta {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int ok() {
  g_err.clear();
  return TA_OK;
}

const char* last_error() { return g_err.c_str(); }

namespace {

int64_t align256(int64_t x) { return (x + 255) & ~(int64_t)255; }
int64_t align32(int64_t x) { return (x + 31) & ~(int64_t)31; }

struct Carver {
  int64_t at = 0;
  int64_t take(int64_t bytes) {
    const int64_t o = at;
    at += align256(bytes);
    return o;
  }
};

bool strides_ok(const int64_t* s) { return s[0] % 8 == 0 && s[1] % 8 == 0 && s[2] % 8 == 0; }

}  // namespace

// Builds and validates the plan; returns TA_OK or an error code (message set).
int make_plan(const ta_problem* p, Plan* P, bool chunk) {
  if (!p) return fail(TA_ERR_INVALID, "problem is NULL");
  P->p = *p;
  const int64_t B = p->B, L = p->L, N = p->N, H = p->H, D = p->D, S = p->num_samples;
  const int64_t b = p->branching, LB = p->leaf_block;
  if (B < 1 || L < 1 || N < 1 || H < 1)
    return fail(TA_ERR_INVALID, "B, L, N, H must be >= 1 (got %lld, %lld, %lld, %lld)", (long long)B, (long long)L,
                (long long)N, (long long)H);
  if (p->causal == TA_CAUSAL_EXACT && L > N)
    return fail(TA_ERR_INVALID, "causal needs L <= N (got L=%lld, N=%lld)", (long long)L, (long long)N);
  if (D != 32 && D != 64 && D != 96 && D != 128)
    return fail(TA_ERR_UNSUPPORTED, "head_dim must be one of 32, 64, 96, 128 (got %lld)", (long long)D);
  if (S < 1 || S > kMaxSamples)
    return fail(TA_ERR_UNSUPPORTED,
                "num_samples must be in [1, %d] for one launch (got %lld); ta_forward and ta_backward take up to %d",
                kMaxSamples, (long long)S, kMaxChunks * kMaxSamples);
  if (b < 2 || b > 64 || (b & (b - 1)))
    return fail(TA_ERR_INVALID, "branching must be a power of two in [2, 64] (got %lld)", (long long)b);
  if (LB < 1 || LB > 128) return fail(TA_ERR_UNSUPPORTED, "leaf_block must be in [1, 128] (got %lld)", (long long)LB);
  if (N % LB) return fail(TA_ERR_INVALID, "N=%lld is not a multiple of leaf_block=%lld", (long long)N, (long long)LB);
  if (p->dtype != TA_F32 && p->dtype != TA_BF16 && p->dtype != TA_F16)
    return fail(TA_ERR_INVALID, "unknown dtype %d", p->dtype);
  if (p->tree_mode != TA_TREE_NATURAL && p->tree_mode != TA_TREE_COMPAT && p->tree_mode != TA_TREE_NODEKEYS)
    return fail(TA_ERR_INVALID, "unknown tree_mode %d", p->tree_mode);
  if (p->tree_mode != TA_TREE_NATURAL && b != 2)
    return fail(TA_ERR_INVALID, "compat and node-key trees are binary (branching=%lld)", (long long)b);
  if (p->tree_mode == TA_TREE_NODEKEYS && LB != 1)
    return fail(TA_ERR_INVALID, "node-key trees have one leaf per position (leaf_block=%lld)", (long long)LB);
  if (p->causal != TA_CAUSAL_NONE && p->causal != TA_CAUSAL_EXACT && p->causal != TA_CAUSAL_REFERENCE)
    return fail(TA_ERR_INVALID, "causal must be TA_CAUSAL_NONE, _EXACT or _REFERENCE (got %d)", p->causal);
  if (p->causal == TA_CAUSAL_REFERENCE && (b != 2 || LB != 1 || p->tree_mode == TA_TREE_NATURAL))
    return fail(TA_ERR_INVALID, "the reference causal mode needs the reference tree: branching 2, leaf_block 1, "
                                "compat or node-key summaries");
  if (!(p->max_logit > 0.f)) return fail(TA_ERR_INVALID, "max_logit must be > 0");
  const int64_t NL = N / LB;
  int T = 0;
  int64_t pw = 1;
  while (pw < NL) {
    pw *= b;
    ++T;
    if (T > kMaxDepth) break;
  }
  if (pw != NL || T > kMaxDepth)
    return fail(TA_ERR_INVALID, "N/leaf_block=%lld must be a power of branching=%lld (depth <= %d)", (long long)NL,
                (long long)b, kMaxDepth);
  if (L * S >= (int64_t)1 << 31) return fail(TA_ERR_UNSUPPORTED, "L*num_samples must be < 2^31");
  if (!strides_ok(p->q_strides) || !strides_ok(p->k_strides) || !strides_ok(p->v_strides) ||
      !strides_ok(p->o_strides) || !strides_ok(p->g_strides))
    return fail(TA_ERR_UNSUPPORTED, "tensor strides must be multiples of 8 elements");

  P->B = B; P->L = L; P->N = N; P->H = H; P->D = D; P->S = S; P->BH = B * H;
  P->s0 = 0;
  P->s_total = S;
  memset(&P->acc, 0, sizeof(P->acc));
  P->esize = p->dtype == TA_F32 ? 4 : 2;
  Geo& G = P->geo;
  memset(&G, 0, sizeof(G));
  G.b = (int)b; G.T = T; G.NL = (int)NL; G.LB = (int)LB;
  G.lb = 0;
  while ((1 << G.lb) < b) ++G.lb;
  G.pw[0] = 1;
  for (int i = 1; i <= T; ++i) G.pw[i] = G.pw[i - 1] * (int)b;
  G.off[0] = 0;
  G.off[1] = 0;
  for (int lam = 1; lam <= T; ++lam) G.off[lam + 1] = G.off[lam] + (int)align32(G.pw[lam]);
  G.NS = G.off[T + 1];
  if ((int64_t)G.NS * D * 4 * P->BH > ((int64_t)1 << 40)) return fail(TA_ERR_UNSUPPORTED, "tree too large");
  // The sampler's level tiles cost O(L * level width); levels with more than
  // kSampleDenseCols children (b = 2 or 4) are evaluated per sampled item instead.
  if (p->dense_cols < 0) return fail(TA_ERR_INVALID, "dense_cols must be >= 0 (got %d)", p->dense_cols);
  // deep binary trees (the reference tree at L >= 16384): levels up to 512
  // children as tiles (sampler 2.92 -> 2.70 ms at L = 16384, 14.0 -> 13.2 ms at 65536)
  const int64_t sdef = (b == 2 && T >= 14) ? 512 : kSampleDenseCols;
  const int64_t scols = p->dense_cols > 0 ? p->dense_cols : sdef;
  P->sample_dense = T;
  if (b == 2 || b == 4)
    for (int d = 0; d < T; ++d)
      if (G.pw[d + 1] > scols) {
        P->sample_dense = d;
        break;
      }
  // Likewise the backward's dense G tiles (and their G^T rows in the
  // workspace) cover levels with at most kTreeDenseCols children; deeper ones
  // run in the band kernels, linear in the sampled pairs.
  // Deep binary trees (the reference tree at L >= 16384) run their widest dense
  // levels in bands too: the tree backward at L = 16384 takes 5.23 ms with
  // levels up to 512 children dense against 6.05 ms up to 1024, and at
  // L = 65536 31.9 ms up to 256 against 38.8 ms up to 1024.
  const int64_t tdef = (b == 2 && T >= 16) ? 256 : (b == 2 && T >= 14) ? 512 : kTreeDenseCols;
  const int64_t tcols = p->dense_cols > 0 ? p->dense_cols : tdef;
  P->tree_dense = T;
  if (b == 2 || b == 4)
    for (int d = 0; d < T; ++d)
      if (G.pw[d + 1] > tcols) {
        P->tree_dense = d;
        break;
      }
  const int64_t NSd = G.off[P->tree_dense + 1];  // dense rows

  // bucketing: one count per (leaf block, chunk of kQueryChunk queries), or
  // with more leaf blocks than one LDS window a radix sort and one count per block
  P->qc = kQueryChunk;
  P->bucket_sort = NL > kBucketWin;
  P->nchunk = P->bucket_sort ? 1 : (int)((L + kQueryChunk - 1) / kQueryChunk);
  if (P->bucket_sort && B * H * (NL + 1) > ((int64_t)1 << 32) - 1)
    return fail(TA_ERR_UNSUPPORTED, "B*H*(N/leaf_block + 1) must be < 2^32 (got %lld)",
                (long long)(B * H * (NL + 1)));
  if (B * L * H * S >= ((int64_t)1 << 32)) return fail(TA_ERR_UNSUPPORTED, "B*L*H*num_samples must be < 2^32");
  if (P->bucket_sort && B * L * H * S >= ((int64_t)1 << 31))
    return fail(TA_ERR_UNSUPPORTED, "with more than %d leaf blocks B*L*H*num_samples must be < 2^31", kBucketWin);
  P->npiece = (int)(NL + (L * S + kPieceFwd - 1) / kPieceFwd);
  if ((int64_t)P->npiece * P->BH > ((int64_t)1 << 31) - 1)
    return fail(TA_ERR_UNSUPPORTED, "too many leaf-forward pieces (NL=%lld)", (long long)NL);
  if ((int64_t)NL * P->nchunk * P->BH > ((int64_t)1 << 29))
    return fail(TA_ERR_UNSUPPORTED, "too many leaf blocks x query chunks for the bucket table (NL=%lld)",
                (long long)NL);
  // summary gradient: chunks of 384 summary rows; queries split into blocks of
  // 64 so the product has about 512 workgroups (two per CU)
  const int64_t qtiles = (L + kQueryTile - 1) / kQueryTile;
  P->Lp = qtiles * kQueryTile;
  const int64_t rowchunks = (NSd / 16 + 23) / 24 > 0 ? (NSd / 16 + 23) / 24 : 1;
  const int64_t kblocks = P->Lp / 64;
  int64_t qsplit = (512 + rowchunks * P->BH - 1) / (rowchunks * P->BH);
  if (qsplit < 1) qsplit = 1;
  if (qsplit > kblocks) qsplit = kblocks;
  P->qsplit = (int)qsplit;

  const int64_t BLHS = B * L * H * S;
  const int64_t es = P->esize;
  const bool half = es == 2;
  // The tree gradient along each pair's path inside the leaf backward (its T*b
  // child rows are one more MFMA tile per pair tile): 16-bit inputs, leaf
  // blocks of two or more tokens, b = 2 or 4 with T*b <= 32, not the
  // reference causal mode, dense_cols at its default, and the leaf tile with
  // the path rows inside the LDS.  Otherwise the dense level tiles and bands.
  P->path_rows = 0;
  if (half && LB > 1 && (b == 2 || b == 4) && T >= 1 && T * b <= 32 && p->causal != TA_CAUSAL_REFERENCE &&
      p->dense_cols == 0) {
    P->path_rows = T * b <= 16 ? 16 : 32;
    if (leaf_bwd_smem(*P) < 0) P->path_rows = 0;
  }
  // One-token leaves (the reference's binary tree), 16-bit, not the reference
  // causal mode, dense_cols at its default: the tree gradient along the paths
  // per subtree of 2^g leaves (leaf_path1.hip), up to 16 depths above them.
  P->leaf_path = 0;
  if (half && LB == 1 && b == 2 && T >= 1 && p->causal != TA_CAUSAL_REFERENCE && p->dense_cols == 0) {
    const int g = leaf_path1_depth(T);
    if (2 * (T - g) <= leaf_path1_top_rows() && leaf_path1_smem((int)D) <= 160 * 1024) P->leaf_path = g;
  }
  const bool pr = P->path_rows > 0, lp = P->leaf_path > 0;
  Carver r;
  P->rec.summaries = r.take(P->BH * G.NS * D * 4);
  P->rec.sum_hi = r.take(half ? P->BH * G.NS * D * es : 0);
  P->rec.sum_lo = r.take(half ? P->BH * G.NS * D * es : 0);
  P->rec.sum_t = r.take(pr || lp ? 0 : P->BH * G.NS * D * es);  // the dense backward's transposed copy
  P->rec.means = r.take(p->tree_mode == TA_TREE_NODEKEYS ? 0 : P->BH * NL * D * 4);
  P->rec.segs = r.take(p->tree_mode == TA_TREE_NODEKEYS || NL < 128 ? 0 : P->BH * (NL / 64 + NL / 4096) * D * 4);
  P->rec.leaf = r.take(BLHS * 4);
  P->rec.slot_leaf = r.take(BLHS * 4);
  P->rec.slot_weight = r.take(BLHS * 4);
  P->rec.slot_count = r.take(B * L * H * 4);
  P->rec.lse = r.take(B * L * H * 4);
  P->rec.hist = r.take(P->BH * NL * P->nchunk * 4);
  P->rec.block_start = r.take(P->BH * (NL + 1) * 4);
  P->rec.order = r.take(P->BH * L * S * 4);
  P->rec.piece_start = r.take(P->BH * (NL + 1) * 4);
  P->rec.piece_block = r.take(P->BH * P->npiece * 4);
  P->nseg = (int)((NL * P->nchunk + 16383) / 16384);  // segments of 1024 threads x 16 counts
  P->rec.seg_sum = r.take(P->BH * P->nseg * 4);
  P->rec.dstar = r.take(p->causal == TA_CAUSAL_REFERENCE ? L * 4 : 0);
  P->rec.logA = r.take(p->causal == TA_CAUSAL_EXACT && P->sample_dense < T ? B * L * H * (T + 1) * 4 : 0);
  // the radix sort's key and value double buffers and per-tile digit counts
  P->rec.sort_keys = r.take(P->bucket_sort ? 2 * BLHS * 4 : 0);
  P->rec.sort_vals = r.take(P->bucket_sort ? 2 * BLHS * 4 : 0);
  P->rec.sort_hist = r.take(P->bucket_sort ? 256 * ((BLHS + 2047) / 2048 + 1) * 4 : 0);
  P->rec.out_e = r.take(pr && !chunk ? B * L * H * D * es : 0);
  P->rec.total = r.at;
  const bool lb1 = LB == 1;  // leaf stage: a value gather, no pair rows
  Carver f;
  P->fws.partial = f.take(lb1 ? 0 : BLHS * D * es);
  P->fws.total = f.at;
  Carver w;
  P->bws.delta = w.take(pr ? 0 : BLHS * 4);
  P->bws.dq_part = w.take(!lb1 || lp || P->tree_dense < T ? BLHS * D * es : 0);
  P->bws.dlogp = w.take(pr ? 0 : BLHS * 4);
  P->bws.dk_leaf = w.take(p->tree_mode == TA_TREE_NODEKEYS || lb1 ? 0 : B * N * H * D * 4);
  P->bws.gt = w.take(pr || lp ? 0 : P->BH * NSd * P->Lp * es);
  P->bws.qt = w.take(pr || lp ? 0 : P->BH * D * P->Lp * es);
  P->bws.dsum_part = w.take(pr || lp ? 0 : qsplit * P->BH * NSd * D * 4);
  P->bws.dsum = w.take(P->BH * G.NS * D * 4);
  P->bws.mean = w.take(pr ? B * L * H * 4 : 0);
  P->bws.dcp = w.take(pr ? P->BH * NL * T * b * D * 4
                         : lp ? P->BH * (NL >> P->leaf_path) * leaf_path1_top_rows() * D * 4 : 0);
  const bool rc = p->causal == TA_CAUSAL_REFERENCE;
  P->bws.rc_coef = w.take(rc ? B * L * H * T * 4 : 0);
  P->bws.rc_rho = w.take(rc ? B * L * H * T * 4 : 0);
  P->bws.rc_g = w.take(rc ? B * L * H * T * 4 : 0);
  P->bws.total = w.at;

  if (rc && ref_sample_smem(*P) > 160 * 1024)
    return fail(TA_ERR_UNSUPPORTED, "the reference causal mode keeps a query's B*H*S lanes in one workgroup; "
                                    "B*H*S=%lld is too large", (long long)(P->BH * S));
  if (leaf_fwd_smem(*P) < 0 || leaf_bwd_smem(*P) < 0)
    return fail(TA_ERR_UNSUPPORTED, "leaf_block=%lld with head_dim=%lld in this dtype exceeds the 160 KiB LDS tile",
                (long long)LB, (long long)D);
  return TA_OK;
}

int make_chunks(const ta_problem* p, Chunks* C) {
  if (!p) return fail(TA_ERR_INVALID, "problem is NULL");
  const int64_t S = p->num_samples;
  if (S <= kMaxSamples) {
    C->n = 1;
    const int rc = make_plan(p, &C->P[0]);
    if (rc) return rc;
    const Plan& P = C->P[0];
    C->rec_off[0] = 0;
    C->rec_leaf = P.rec.leaf;
    C->rec_out32 = -1;
    C->rec_total = P.rec.total;
    C->fws_total = P.fws.total;
    C->bws_dq32 = C->bws_dv32 = C->bws_dkl = C->bws_dsum = C->bws_mean = -1;
    C->bws_chunk = 0;
    C->bws_total = P.bws.total;
    return TA_OK;
  }
  if (S > (int64_t)kMaxChunks * kMaxSamples)
    return fail(TA_ERR_UNSUPPORTED, "num_samples must be in [1, %d] (got %lld)", kMaxChunks * kMaxSamples,
                (long long)S);
  if (p->causal == TA_CAUSAL_REFERENCE)
    return fail(TA_ERR_UNSUPPORTED, "the reference causal mode couples every sample of a query in one workgroup; "
                                    "num_samples must be <= %d there (got %lld)", kMaxSamples, (long long)S);
  const int n = (int)((S + kMaxSamples - 1) / kMaxSamples);
  C->n = n;
  Carver r, w;
  int64_t fws = 0, bws = 0, s0 = 0;
  for (int g = 0; g < n; ++g) {
    ta_problem pg = *p;
    pg.num_samples = S / n + (g < S % n ? 1 : 0);
    const int rc = make_plan(&pg, &C->P[g], true);
    if (rc) return rc;
    Plan& P = C->P[g];
    P.s0 = s0;
    P.s_total = S;
    s0 += pg.num_samples;
    C->rec_off[g] = r.take(P.rec.total);
    fws = fws > P.fws.total ? fws : P.fws.total;
    bws = bws > P.bws.total ? bws : P.bws.total;
  }
  const Plan& P0 = C->P[0];
  const int64_t BLH = P0.B * P0.L * P0.H, BNH = P0.B * P0.N * P0.H, D = P0.D;
  C->rec_leaf = r.take(BLH * S * 4);
  C->rec_out32 = r.take(BLH * D * 4);
  C->rec_total = r.at;
  C->fws_total = fws;
  C->bws_dq32 = w.take(BLH * D * 4);
  C->bws_dv32 = w.take(BNH * D * 4);
  const bool dkl = P0.geo.LB > 1 && p->tree_mode != TA_TREE_NODEKEYS;  // the leaf stage has a dk part
  C->bws_dkl = w.take(dkl ? BNH * D * 4 : 0);
  C->bws_dsum = w.take(P0.BH * P0.geo.NS * D * 4);
  C->bws_mean = w.take(BLH * 4);
  C->bws_chunk = w.take(bws);
  C->bws_total = w.at;
  return TA_OK;
}

namespace {

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int launch_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(TA_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

}  // namespace
}  // namespace ta

namespace ta {
namespace {

// Forward of a problem with more samples than one launch: every chunk's pool
// and sampler, the merge of the chunks' normalizers, then every chunk's
// bucketing and leaf stage adding into the float output, rounded once.
int forward_chunks(const ta_problem* p, const void* q, const void* k, const void* v, const float* U, uint64_t seed,
                   const uint8_t* packed, void* out, float* weights, void* record, void* workspace, void* stream) {
  static thread_local Chunks C;
  int rc = make_chunks(p, &C);
  if (rc) return rc;
  const bool need_k = p->tree_mode != TA_TREE_NODEKEYS;
  const bool need_ws = C.fws_total > 0;  // leaf_block 1 needs none
  if (!q || !v || !out || !weights || !record || (need_ws && !workspace) || (need_k && !k) || !aligned16(q) ||
      !aligned16(v) || !aligned16(out) || !aligned16(record) || !aligned16(workspace) || (need_k && !aligned16(k)))
    return fail(TA_ERR_INVALID, "q/k/v/out/weights/record/workspace must be 16-byte aligned device pointers");
  hipStream_t st = (hipStream_t)stream;
  char* rec = (char*)record;
  ChunkRecs R;
  R.n = C.n;
  for (int g = 0; g < C.n; ++g) {
    const Plan& P = C.P[g];
    char* rg = rec + C.rec_off[g];
    hipError_t e = launch_pool(P, k, rg, st);
    if (e != hipSuccess) return launch_status(e, "pool");
    e = launch_sample(P, q, U, seed, weights + P.s0, rg, st, packed);
    if (e != hipSuccess) return launch_status(e, packed ? "replay" : "sample");
    R.S[g] = (int)P.S;
    R.s0[g] = (int)P.s0;
    R.lse[g] = (const float*)(rg + P.rec.lse);
    R.slot_weight[g] = (float*)(rg + P.rec.slot_weight);
    R.slot_count[g] = (const int*)(rg + P.rec.slot_count);
    R.leaf[g] = (const int*)(rg + P.rec.leaf);
  }
  hipError_t e = launch_chunk_merge(C.P[0], R, weights, (int*)(rec + C.rec_leaf), st);
  if (e != hipSuccess) return launch_status(e, "chunk_merge");
  float* out32 = (float*)(rec + C.rec_out32);
  for (int g = 0; g < C.n; ++g) {
    Plan P = C.P[g];
    char* rg = rec + C.rec_off[g];
    e = launch_bucket(P, rg, st);
    if (e != hipSuccess) return launch_status(e, "bucket");
    P.acc.out32 = out32;
    P.acc.first = g == 0;
    e = launch_leaf_fwd(P, q, k, v, out, rg, (char*)workspace, st);
    if (e != hipSuccess) return launch_status(e, "leaf_forward");
  }
  const Plan& P0 = C.P[0];
  return launch_status(launch_cast_rows(p->dtype, out32, out, p->o_strides, P0.B, P0.L, P0.H, P0.D, st), "cast");
}

// Backward of a chunked problem: mean = dout . out over all samples, then per
// chunk the leaf and tree backward (dl_u = W_u (delta_u - mean), W the
// weights over all samples) adding into float accumulators; the last chunk
// runs the key adjoint from the summed leaf dk and summary gradient.
int backward_chunks(const ta_problem* p, const void* q, const void* k, const void* v, const void* grad_out,
                    const float* weights, const void* record, void* dq, void* dk, void* dv, void* workspace,
                    void* stream) {
  static thread_local Chunks C;
  int rc = make_chunks(p, &C);
  if (rc) return rc;
  const bool need_k = p->tree_mode != TA_TREE_NODEKEYS;
  if (!q || !v || !grad_out || !weights || !record || !dq || !dk || !dv || !workspace || (need_k && !k))
    return fail(TA_ERR_INVALID, "NULL device pointer");
  const void* al[] = {q, v, grad_out, record, dq, dk, dv, workspace};
  for (const void* x : al)
    if (!aligned16(x)) return fail(TA_ERR_INVALID, "device pointers must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  const char* rec = (const char*)record;
  char* ws = (char*)workspace;
  ChunkAcc acc;
  acc.out32 = nullptr;
  acc.dq32 = (float*)(ws + C.bws_dq32);
  acc.dv32 = (float*)(ws + C.bws_dv32);
  acc.dk_leaf = (float*)(ws + C.bws_dkl);
  acc.dsum = (float*)(ws + C.bws_dsum);
  acc.mean = (const float*)(ws + C.bws_mean);
  const Plan& P0 = C.P[0];
  hipError_t e = launch_chunk_mean(P0, grad_out, rec + C.rec_out32, false, (float*)(ws + C.bws_mean), st);
  if (e != hipSuccess) return launch_status(e, "chunk_mean");
  for (int g = 0; g < C.n; ++g) {
    Plan P = C.P[g];
    P.acc = acc;
    P.acc.first = g == 0;
    P.acc.last = g == C.n - 1;
    const char* rg = rec + C.rec_off[g];
    char* wg = ws + C.bws_chunk;
    e = launch_leaf_bwd(P, q, k, v, grad_out, rg, dv, wg, st);
    if (e != hipSuccess) return launch_status(e, "leaf_backward");
    e = launch_tree_bwd(P, q, weights, rg, dq, dk, wg, st);
    if (e != hipSuccess) return launch_status(e, "tree_backward");
  }
  e = launch_cast_rows(p->dtype, acc.dq32, dq, p->q_strides, P0.B, P0.L, P0.H, P0.D, st);
  if (e != hipSuccess) return launch_status(e, "cast");
  return launch_status(launch_cast_rows(p->dtype, acc.dv32, dv, p->v_strides, P0.B, P0.N, P0.H, P0.D, st), "cast");
}

}  // namespace
}  // namespace ta

using namespace ta;

extern "C" {

int ta_version(void) { return TA_VERSION; }

const char* ta_last_error(void) { return last_error(); }

int ta_record_bytes(const ta_problem* p, int64_t* bytes) {
  static thread_local Chunks C;
  const int rc = make_chunks(p, &C);
  if (rc) return rc;
  if (!bytes) return fail(TA_ERR_INVALID, "bytes is NULL");
  *bytes = C.rec_total;
  return ok();
}

int ta_forward_workspace_bytes(const ta_problem* p, int64_t* bytes) {
  static thread_local Chunks C;
  const int rc = make_chunks(p, &C);
  if (rc) return rc;
  if (!bytes) return fail(TA_ERR_INVALID, "bytes is NULL");
  *bytes = C.fws_total;
  return ok();
}

int ta_backward_workspace_bytes(const ta_problem* p, int64_t* bytes) {
  static thread_local Chunks C;
  const int rc = make_chunks(p, &C);
  if (rc) return rc;
  if (!bytes) return fail(TA_ERR_INVALID, "bytes is NULL");
  *bytes = C.bws_total;
  return ok();
}

int ta_record_offset(const ta_problem* p, int which, int64_t* offset) {
  static thread_local Chunks C;
  const int rc = make_chunks(p, &C);
  if (rc) return rc;
  if (!offset) return fail(TA_ERR_INVALID, "offset is NULL");
  const Plan& P = C.P[0];
  switch (which) {
    case TA_REC_LEAVES: *offset = C.rec_leaf; break;
    case TA_REC_SUMMARIES: *offset = C.rec_off[0] + P.rec.summaries; break;
    case TA_REC_NUM_ROWS: *offset = P.geo.NS; break;
    default: return fail(TA_ERR_INVALID, "unknown record piece %d", which);
  }
  return ok();
}

int ta_fill_uniforms(uint64_t seed, int64_t n, float* out, void* stream) {
  if (n < 0 || (n > 0 && !out)) return fail(TA_ERR_INVALID, "bad uniform buffer");
  return launch_status(launch_fill_uniforms(seed, n, out, (hipStream_t)stream), "fill_uniforms");
}

int ta_pool(const ta_problem* p, const void* k, void* record, void* stream) {
  Plan P;
  const int rc = make_plan(p, &P);
  if (rc) return rc;
  if (!k || !record || !aligned16(k) || !aligned16(record)) return fail(TA_ERR_INVALID, "k/record must be 16-byte aligned device pointers");
  return launch_status(launch_pool(P, k, (char*)record, (hipStream_t)stream), "pool");
}

int ta_sample(const ta_problem* p, const void* q, const float* uniforms, uint64_t seed, float* weights, void* record,
              void* stream) {
  Plan P;
  const int rc = make_plan(p, &P);
  if (rc) return rc;
  if (!q || !weights || !record || !aligned16(q) || !aligned16(record))
    return fail(TA_ERR_INVALID, "q/weights/record must be device pointers (q, record 16-byte aligned)");
  return launch_status(launch_sample(P, q, uniforms, seed, weights, (char*)record, (hipStream_t)stream), "sample");
}

int ta_bucket(const ta_problem* p, void* record, void* stream) {
  Plan P;
  const int rc = make_plan(p, &P);
  if (rc) return rc;
  if (!record || !aligned16(record)) return fail(TA_ERR_INVALID, "record must be a 16-byte aligned device pointer");
  return launch_status(launch_bucket(P, (char*)record, (hipStream_t)stream), "bucket");
}

int ta_leaf_forward(const ta_problem* p, const void* q, const void* k, const void* v, void* out, void* record,
                    void* workspace, void* stream) {
  Plan P;
  const int rc = make_plan(p, &P);
  if (rc) return rc;
  const bool need_k = p->tree_mode != TA_TREE_NODEKEYS;
  const bool need_ws = P.fws.total > 0;  // leaf_block 1 needs none
  if (!q || !v || !out || !record || (need_ws && !workspace) || (need_k && !k) || !aligned16(q) || !aligned16(v) ||
      !aligned16(out) || !aligned16(record) || !aligned16(workspace) || (need_k && !aligned16(k)))
    return fail(TA_ERR_INVALID, "q/k/v/out/record/workspace must be 16-byte aligned device pointers");
  return launch_status(launch_leaf_fwd(P, q, k, v, out, (char*)record, (char*)workspace, (hipStream_t)stream),
                       "leaf_forward");
}

int ta_forward(const ta_problem* p, const void* q, const void* k, const void* v, const float* uniforms, uint64_t seed,
               void* out, float* weights, void* record, void* workspace, void* stream) {
  if (p && p->num_samples <= kMaxSamples) {
    int rc = ta_pool(p, k, record, stream);
    if (rc) return rc;
    rc = ta_sample(p, q, uniforms, seed, weights, record, stream);
    if (rc) return rc;
    rc = ta_bucket(p, record, stream);
    if (rc) return rc;
    return ta_leaf_forward(p, q, k, v, out, record, workspace, stream);
  }
  return forward_chunks(p, q, k, v, uniforms, seed, nullptr, out, weights, record, workspace, stream);
}

int ta_leaf_backward(const ta_problem* p, const void* q, const void* k, const void* v, const void* grad_out,
                     const void* record, void* dv, void* workspace, void* stream) {
  Plan P;
  const int rc = make_plan(p, &P);
  if (rc) return rc;
  const bool need_k = p->tree_mode != TA_TREE_NODEKEYS;
  if (!q || !v || !grad_out || !record || !dv || !workspace || (need_k && !k))
    return fail(TA_ERR_INVALID, "NULL device pointer");
  const void* al[] = {q, v, grad_out, record, dv, workspace};
  for (const void* x : al)
    if (!aligned16(x)) return fail(TA_ERR_INVALID, "device pointers must be 16-byte aligned");
  if (need_k && !aligned16(k)) return fail(TA_ERR_INVALID, "device pointers must be 16-byte aligned");
  return launch_status(launch_leaf_bwd(P, q, k, v, grad_out, (const char*)record, dv, (char*)workspace,
                                       (hipStream_t)stream),
                       "leaf_backward");
}

int ta_tree_backward(const ta_problem* p, const void* q, const float* weights, const void* record, void* dq, void* dk,
                     void* workspace, void* stream) {
  Plan P;
  const int rc = make_plan(p, &P);
  if (rc) return rc;
  if (!q || !weights || !record || !dq || !dk || !workspace) return fail(TA_ERR_INVALID, "NULL device pointer");
  const void* al[] = {q, record, dq, dk, workspace};
  for (const void* x : al)
    if (!aligned16(x)) return fail(TA_ERR_INVALID, "device pointers must be 16-byte aligned");
  return launch_status(
      launch_tree_bwd(P, q, weights, (const char*)record, dq, dk, (char*)workspace, (hipStream_t)stream),
      "tree_backward");
}

int ta_backward(const ta_problem* p, const void* q, const void* k, const void* v, const void* grad_out,
                const float* weights, const void* record, void* dq, void* dk, void* dv, void* workspace,
                void* stream) {
  if (p && p->num_samples > kMaxSamples)
    return backward_chunks(p, q, k, v, grad_out, weights, record, dq, dk, dv, workspace, stream);
  Plan P;
  const int rc = make_plan(p, &P);
  if (rc) return rc;
  const bool need_k = p->tree_mode != TA_TREE_NODEKEYS;
  if (!q || !v || !grad_out || !weights || !record || !dq || !dk || !dv || !workspace || (need_k && !k))
    return fail(TA_ERR_INVALID, "NULL device pointer");
  const void* al[] = {q, v, grad_out, record, dq, dk, dv, workspace};
  for (const void* x : al)
    if (!aligned16(x)) return fail(TA_ERR_INVALID, "device pointers must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = launch_leaf_bwd(P, q, k, v, grad_out, (const char*)record, dv, (char*)workspace, st);
  if (e != hipSuccess) return launch_status(e, "leaf_backward");
  return launch_status(launch_tree_bwd(P, q, weights, (const char*)record, dq, dk, (char*)workspace, st),
                       "tree_backward");
}

// ---- deterministic mode

static int det_depth(int64_t N, int* T) {
  if (N < 2 || N > TA_DET_MAX_LEAVES || (N & (N - 1)))
    return fail(TA_ERR_UNSUPPORTED, "deterministic mode needs N = 2^T leaves with 2 <= N <= %d (got %lld)",
                TA_DET_MAX_LEAVES, (long long)N);
  int t = 0;
  while ((1LL << t) < N) ++t;
  *T = t;
  return TA_OK;
}

int ta_det_weights(const float* X, int64_t ldx, float* W, int64_t ldw, int64_t rows, int64_t L, int64_t N, int causal,
                   void* stream) {
  int T = 0;
  const int rc = det_depth(N, &T);
  if (rc) return rc;
  if (rows < 0 || L < 1 || rows % L) return fail(TA_ERR_INVALID, "rows must be a multiple of L >= 1");
  if (ldx < N - 1 || ldw < N) return fail(TA_ERR_INVALID, "row strides too small (ldx >= N-1, ldw >= N)");
  if (rows > 0 && (!X || !W)) return fail(TA_ERR_INVALID, "NULL device pointer");
  if (rows >= ((int64_t)1 << 31)) return fail(TA_ERR_UNSUPPORTED, "too many rows");
  if (rows == 0) return ok();
  return launch_status(launch_det_weights(X, ldx, W, ldw, rows, (int)L, (int)N, T, causal != 0, (hipStream_t)stream),
                       "det_weights");
}

int ta_det_grad(float* XG, int64_t ldx, const float* W, const float* dW, int64_t ldw, int64_t rows, int64_t N,
                int causal, void* stream) {
  int T = 0;
  const int rc = det_depth(N, &T);
  if (rc) return rc;
  if (rows < 0) return fail(TA_ERR_INVALID, "rows must be >= 0");
  if (ldx < N - 1 || ldw < N) return fail(TA_ERR_INVALID, "row strides too small (ldx >= N-1, ldw >= N)");
  if (rows > 0 && (!XG || !W || !dW)) return fail(TA_ERR_INVALID, "NULL device pointer");
  if (rows >= ((int64_t)1 << 31)) return fail(TA_ERR_UNSUPPORTED, "too many rows");
  if (rows == 0) return ok();
  return launch_status(launch_det_grad(XG, ldx, W, dW, ldw, rows, (int)N, T, causal != 0, (hipStream_t)stream),
                       "det_grad");
}

static int haar_check(int dtype, const void* a, const void* b, const int64_t* s, int64_t B, int64_t H, int64_t D,
                      int64_t N) {
  if (dtype != TA_F32 && dtype != TA_BF16 && dtype != TA_F16) return fail(TA_ERR_INVALID, "unknown dtype %d", dtype);
  if (B < 1 || H < 1 || N < 2 || (N & (N - 1))) return fail(TA_ERR_INVALID, "need B, H >= 1 and N = 2^T >= 2");
  if (D < 4 || D % 4) return fail(TA_ERR_UNSUPPORTED, "head_dim must be a multiple of 4 (got %lld)", (long long)D);
  if (!a || !b || !s) return fail(TA_ERR_INVALID, "NULL pointer");
  if (((uintptr_t)a & 15) || ((uintptr_t)b & 15)) return fail(TA_ERR_INVALID, "pointers must be 16-byte aligned");
  if (N * B * H * D >= ((int64_t)1 << 40)) return fail(TA_ERR_UNSUPPORTED, "tensor too large");
  return TA_OK;
}

int ta_haar_workspace_bytes(int64_t B, int64_t H, int64_t D, int64_t N, int64_t* bytes) {
  if (!bytes) return fail(TA_ERR_INVALID, "NULL output");
  if (B < 1 || H < 1 || N < 2 || (N & (N - 1)) || D < 4 || D % 4)
    return fail(TA_ERR_INVALID, "need B, H >= 1, N = 2^T >= 2 and D a multiple of 4");
  *bytes = 4 * haar_workspace_floats((int)B, (int)H, (int)D, (int)N);
  return ok();
}

int ta_haar_keys(int dtype, const void* k, const int64_t* k_strides, float* out, float* workspace, int64_t B,
                 int64_t H, int64_t D, int64_t N, void* stream) {
  const int rc = haar_check(dtype, k, out, k_strides, B, H, D, N);
  if (rc) return rc;
  if (workspace && ((uintptr_t)workspace & 15)) return fail(TA_ERR_INVALID, "workspace must be 16-byte aligned");
  return launch_status(launch_haar_keys(dtype, k, k_strides, out, workspace, (int)B, (int)H, (int)D, (int)N,
                                        (hipStream_t)stream),
                       "haar_keys");
}

int ta_haar_keys_adjoint(int dtype, const float* dkey, void* dk, const int64_t* dk_strides, int64_t B, int64_t H,
                         int64_t D, int64_t N, void* stream) {
  const int rc = haar_check(dtype, dkey, dk, dk_strides, B, H, D, N);
  if (rc) return rc;
  int T = 0;
  while ((1LL << T) < N) ++T;
  return launch_status(launch_haar_keys_adjoint(dtype, dkey, dk, dk_strides, (int)B, (int)H, (int)D, (int)N, T,
                                                (hipStream_t)stream),
                       "haar_keys_adjoint");
}

int ta_det_stream_forward(int dtype, const void* q, const int64_t* q_strides, const void* knodes,
                          const int64_t* k_strides, const void* v, const int64_t* v_strides, void* out,
                          const int64_t* o_strides, float* lse, int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                          int causal, void* stream) {
  int T = 0;
  const int rc = det_depth(N, &T);
  if (rc) return rc;
  if (dtype != TA_BF16 && dtype != TA_F16)
    return fail(TA_ERR_UNSUPPORTED, "the streaming deterministic forward takes bfloat16 / float16 inputs");
  if (N < 64) return fail(TA_ERR_UNSUPPORTED, "the streaming deterministic forward needs N >= 64 (got %lld)", (long long)N);
  if (D != 32 && D != 64 && D != 96 && D != 128)
    return fail(TA_ERR_UNSUPPORTED, "head dim must be 32, 64, 96 or 128 (got %lld)", (long long)D);
  if (B < 0 || L < 0 || H < 0 || B * H >= 65536 || L >= ((int64_t)1 << 30))
    return fail(TA_ERR_INVALID, "bad batch / length / head count");
  if (B * L * H == 0) return ok();
  if (!q || !knodes || !v || !out || !q_strides || !k_strides || !v_strides || !o_strides)
    return fail(TA_ERR_INVALID, "NULL pointer");
  const void* al[] = {q, knodes, v, out};
  for (const void* x : al)
    if (!aligned16(x)) return fail(TA_ERR_INVALID, "device pointers must be 16-byte aligned");
  const int64_t* st[] = {q_strides, k_strides, v_strides, o_strides};
  for (const int64_t* s : st)
    for (int i = 0; i < 3; ++i)
      if (s[i] % 8) return fail(TA_ERR_INVALID, "strides must be multiples of 8 elements");
  return launch_status(launch_det_stream_fwd(dtype, q, q_strides, knodes, k_strides, v, v_strides, out, o_strides, lse,
                                             (int)B, (int)L, (int)H, (int)D, T, causal != 0, (hipStream_t)stream),
                       "det_stream_forward");
}

int ta_det_stream_backward(int dtype, const void* q, const int64_t* q_strides, const void* grad_out,
                           const int64_t* g_strides, const void* knodes, const int64_t* k_strides, const void* v,
                           const int64_t* v_strides, const float* lse, const float* delta, float* dq_sub,
                           float* chunk_totals, float* dknodes, void* dv, const int64_t* dv_strides, int64_t B,
                           int64_t L, int64_t H, int64_t D, int64_t N, int causal, void* stream) {
  int T = 0;
  const int rc = det_depth(N, &T);
  if (rc) return rc;
  if (dtype != TA_BF16 && dtype != TA_F16)
    return fail(TA_ERR_UNSUPPORTED, "the streaming deterministic backward takes bfloat16 / float16 inputs");
  if (N < 64) return fail(TA_ERR_UNSUPPORTED, "the streaming deterministic backward needs N >= 64 (got %lld)", (long long)N);
  if (D != 32 && D != 64 && D != 96 && D != 128)
    return fail(TA_ERR_UNSUPPORTED, "head dim must be 32, 64, 96 or 128 (got %lld)", (long long)D);
  if (B < 0 || L < 0 || H < 0 || B * H >= 65536 || L >= ((int64_t)1 << 30))
    return fail(TA_ERR_INVALID, "bad batch / length / head count");
  if (B * H == 0) return ok();
  if (!q || !grad_out || !knodes || !v || !dq_sub || !chunk_totals || !dknodes || !dv || !q_strides || !g_strides ||
      !k_strides || !v_strides || !dv_strides || (causal && (!lse || !delta)))
    return fail(TA_ERR_INVALID, "NULL pointer");
  const void* al[] = {q, grad_out, knodes, v, dv};
  for (const void* x : al)
    if (!aligned16(x)) return fail(TA_ERR_INVALID, "device pointers must be 16-byte aligned");
  const int64_t* st[] = {q_strides, g_strides, k_strides, v_strides, dv_strides};
  for (const int64_t* s : st)
    for (int i = 0; i < 3; ++i)
      if (s[i] % 8) return fail(TA_ERR_INVALID, "strides must be multiples of 8 elements");
  return launch_status(launch_det_stream_bwd(dtype, q, q_strides, grad_out, g_strides, knodes, k_strides, v,
                                             v_strides, lse, delta, dq_sub, chunk_totals, dknodes, dv, dv_strides,
                                             (int)B, (int)L, (int)H, (int)D, T, causal != 0, (hipStream_t)stream),
                       "det_stream_backward");
}

// ---- packed path record

static int path_nbits(int64_t NL, int* nbits) {
  if (NL < 1 || NL > ((int64_t)1 << 31) || (NL & (NL - 1)))
    return fail(TA_ERR_INVALID, "num_leaf_blocks must be a power of two in [1, 2^31] (got %lld)", (long long)NL);
  int t = 0;
  while (((int64_t)1 << t) < NL) ++t;
  *nbits = t;
  return TA_OK;
}

static int path_dims(int64_t B, int64_t L, int64_t H, int64_t S) {
  if (B < 0 || L < 0 || H < 0 || S < 0) return fail(TA_ERR_INVALID, "negative path dimension");
  if (B * L * H * S >= ((int64_t)1 << 40)) return fail(TA_ERR_UNSUPPORTED, "too many paths");
  return TA_OK;
}

int ta_path_bytes(int64_t num_leaf_blocks, int64_t* bytes) {
  int nb = 0;
  const int rc = path_nbits(num_leaf_blocks, &nb);
  if (rc) return rc;
  if (!bytes) return fail(TA_ERR_INVALID, "NULL output");
  *bytes = (nb + 7) / 8;
  return ok();
}

int ta_pack_paths(const int32_t* leaf, const int64_t* leaf_strides, int64_t B, int64_t L, int64_t H, int64_t S,
                  int64_t num_leaf_blocks, uint8_t* packed, void* stream) {
  int nb = 0;
  int rc = path_nbits(num_leaf_blocks, &nb);
  if (rc) return rc;
  rc = path_dims(B, L, H, S);
  if (rc) return rc;
  if (B * L * H * S > 0 && nb > 0 && (!leaf || !leaf_strides || !packed))
    return fail(TA_ERR_INVALID, "NULL pointer");
  return launch_status(launch_pack_paths(leaf, leaf_strides, B, L, H, S, nb, packed, (hipStream_t)stream),
                       "pack_paths");
}

int ta_unpack_paths(const uint8_t* packed, int64_t B, int64_t L, int64_t H, int64_t S, int64_t num_leaf_blocks,
                    int32_t* leaf, const int64_t* leaf_strides, void* stream) {
  int nb = 0;
  int rc = path_nbits(num_leaf_blocks, &nb);
  if (rc) return rc;
  rc = path_dims(B, L, H, S);
  if (rc) return rc;
  if (B * L * H * S > 0 && (!leaf || !leaf_strides || (nb > 0 && !packed))) return fail(TA_ERR_INVALID, "NULL pointer");
  return launch_status(launch_unpack_paths(packed, B, L, H, S, nb, leaf, leaf_strides, (hipStream_t)stream),
                       "unpack_paths");
}

int ta_replay(const ta_problem* p, const void* q, const uint8_t* packed, float* weights, void* record,
              void* stream) {
  Plan P;
  const int rc = make_plan(p, &P);
  if (rc) return rc;
  if (p->causal != TA_CAUSAL_NONE)
    return fail(TA_ERR_UNSUPPORTED, "path replay is for non-causal problems (as the reference's replay)");
  if (!q || !weights || !record || !aligned16(q) || !aligned16(record) || (P.geo.T > 0 && !packed))
    return fail(TA_ERR_INVALID, "q/packed/weights/record must be device pointers (q, record 16-byte aligned)");
  return launch_status(launch_sample(P, q, nullptr, 0, weights, (char*)record, (hipStream_t)stream, packed),
                       "replay");
}

int ta_forward_replay(const ta_problem* p, const void* q, const void* k, const void* v, const uint8_t* packed,
                      void* out, float* weights, void* record, void* workspace, void* stream) {
  if (p && p->num_samples > kMaxSamples) {
    if (p->causal != TA_CAUSAL_NONE)
      return fail(TA_ERR_UNSUPPORTED, "path replay is for non-causal problems (as the reference's replay)");
    if (!packed) return fail(TA_ERR_INVALID, "packed paths must be a device pointer");
    return forward_chunks(p, q, k, v, nullptr, 0, packed, out, weights, record, workspace, stream);
  }
  int rc = ta_pool(p, k, record, stream);
  if (rc) return rc;
  rc = ta_replay(p, q, packed, weights, record, stream);
  if (rc) return rc;
  rc = ta_bucket(p, record, stream);
  if (rc) return rc;
  return ta_leaf_forward(p, q, k, v, out, record, workspace, stream);
}

}  // extern "C"
