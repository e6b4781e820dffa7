/*
 * treeattn_amd.h -- C ABI of the MI355X (gfx950) tree-attention library (stochastic and
 * deterministic modes).
 *
 * Plain C: pointers, sizes and a HIP stream.  No torch types cross this
 * boundary.  The caller allocates every buffer (outputs, the saved record and
 * the workspaces, sized by the *_bytes queries below); the library never
 * allocates, frees or synchronizes, and launches only on the stream it is
 * given.  Every entry point returns TA_OK or an error code; the message of the
 * last error on the calling thread is available from ta_last_error().
 *
 * Tensors q/k/v/out/dq/dk/dv are 4-D with the last (head) dimension
 * contiguous; their other three strides (batch, position, head) are given in
 * elements, so both the adapters' bshd layout (B,L,H,D) and the op-level
 * (L,B,H,D) layout are read in place.
 *
 * Reference interfaces (paths under the reference repository):
 *   packages/treeattn-cuda/csrc/treeattn_cuda.cpp          (pybind entry points)
 *   packages/treeattn-cuda/src/treeattn_cuda/_autograd.py   (autograd Function)
 *   packages/attn-bench/src/attn_bench/baselines/_treeattn_common.py (Haar keys)
 */
#ifndef TREEATTN_AMD_H
#define TREEATTN_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TA_VERSION 1

/* return codes */
#define TA_OK 0
#define TA_ERR_INVALID 1      /* bad shape / option / pointer */
#define TA_ERR_UNSUPPORTED 2  /* valid request outside what the kernels implement */
#define TA_ERR_LAUNCH 3       /* HIP launch error */

/* element types of q/k/v/out and their gradients */
#define TA_F32 0
#define TA_BF16 1
#define TA_F16 2

/* causal semantics (ta_problem.causal) */
#define TA_CAUSAL_NONE 0
#define TA_CAUSAL_EXACT 1     /* bottom-right aligned (query t sees tokens <= t + N - L, needs
                                 L <= N); sampling is restricted exactly to allowed leaf blocks */
#define TA_CAUSAL_REFERENCE 2 /* the reference's causal stochastic mode (_tree_mha.py:125-268,
                                 379-394): binary trees with leaf_block 1 (compat / node keys),
                                 query t's boundary is leaf t; while every (batch, head, sample)
                                 lane of a query is on the boundary path the decisions are
                                 corrected by the boundary log-masses (fully allowed subtrees
                                 weigh their leaf count), afterwards they are not; when
                                 L > num_samples, queries t < num_samples get exact causal
                                 attention (all leaves n <= t, softmax of the path log-probs) */

/* how the per-node child summaries are built from `k` */
#define TA_TREE_NATURAL 0  /* child summary = mean key of the child's subtree / 2 */
#define TA_TREE_COMPAT 1   /* reference layout: in-order Haar of block means, read in heap order */
#define TA_TREE_NODEKEYS 2 /* `k` already holds the NL-1 heap-ordered node keys (op-level API) */

typedef struct ta_problem {
  int64_t B, L, H, D;    /* batch, query positions, heads, head dim */
  int64_t N;             /* leaf tokens (keys/values); N = leaf_block * b^T.  Causal masks are
                            bottom-right aligned: query t sees tokens <= t + N - L (needs L <= N) */
  int64_t num_samples;   /* S: sampled paths per query, 1..64 for every entry point; ta_forward,
                            ta_forward_replay and ta_backward take up to 1024 (non-reference
                            causal modes), drawn and used in chunks of at most 64 */
  int64_t branching;     /* b >= 2 */
  int64_t leaf_block;    /* LB >= 1 */
  int32_t tree_mode;     /* TA_TREE_* */
  int32_t causal;        /* TA_CAUSAL_* */
  int32_t dtype;         /* TA_F32 / TA_BF16 / TA_F16 */
  int32_t dense_cols;    /* tree levels with at most this many children run as dense level
                            tiles, wider ones per sampled path (0: the library's defaults,
                            which for 16-bit inputs with b = 2 or 4, leaf_block >= 2 and
                            T*b <= 32 take the backward's tree part along the sampled paths
                            in the leaf backward, and for 16-bit one-token binary leaves
                            outside the reference causal mode per subtree of 64 leaves);
                            changes no result beyond rounding, for tuning and tests */
  float scale;           /* leaf-block softmax scale */
  float max_logit;       /* child logits are clamped to +-max_logit/2 (binary compat trees:
                            the left/right logit to +-max_logit, _autograd.py:202) */
  int64_t q_strides[3];  /* (batch, position, head) element strides; also dq */
  int64_t k_strides[3];  /* (batch, token, head) of k and dk; TA_TREE_NODEKEYS: (batch, node, head) */
  int64_t v_strides[3];  /* (batch, token, head) of v and dv */
  int64_t o_strides[3];  /* of out */
  int64_t g_strides[3];  /* of the incoming output gradient */
  int64_t w_strides[3];  /* of the weights (batch, position, head); samples contiguous */
} ta_problem;

/* Library version (TA_VERSION). */
int ta_version(void);

/* Message of the last error returned on this thread ("" if none). */
const char* ta_last_error(void);

/* Sizes of the caller-allocated buffers.  `record` is written by the forward
 * and read by the backward (the Function's saved state); the workspaces are
 * scratch for one call each.  Replaces the reference's torch-side allocations
 * in _autograd.py:685-700 (packed path bits + sampled indices). */
int ta_record_bytes(const ta_problem* p, int64_t* bytes);
int ta_forward_workspace_bytes(const ta_problem* p, int64_t* bytes);
int ta_backward_workspace_bytes(const ta_problem* p, int64_t* bytes);

/* Byte offset of a piece of the record, for callers that read the sampled
 * paths (the reference returns them from its sampler,
 * _autograd.py:223-257):
 *   TA_REC_LEAVES     int32 (B, L, H, S): leaf block sampled by each path;
 *   TA_REC_SUMMARIES  float32 (B*H, NS, D): child summaries, level-major with
 *                     level lam (1..T) at rows sum_{m<lam} roundup32(b^m)
 *                     (NS from TA_REC_NUM_ROWS, returned in *offset). */
#define TA_REC_LEAVES 0
#define TA_REC_SUMMARIES 1
#define TA_REC_NUM_ROWS 2
int ta_record_offset(const ta_problem* p, int which, int64_t* offset);

/* Fill `out[0..n)` with the counter-RNG uniforms in (0,1) that the sampler
 * uses when no uniform tensor is supplied (Philox4x32-10, key = seed).
 * Replaces torch's exponential_() stream (_tree_mha.py:109,
 * sample_non_causal_paths.cu:31-52) with a reproducible one. */
int ta_fill_uniforms(uint64_t seed, int64_t n, float* out, void* stream);

/* Per-level key summaries into the record.  Replaces haar_internal_node_keys
 * (_treeattn_common.py:54-86) and the key re-layout in _tree_mha.py:359-365. */
int ta_pool(const ta_problem* p, const void* k, void* record, void* stream);

/* Path sampling for every (batch, position, head): one wavefront per query
 * walks root->leaf over MFMA child-logit tiles with Gumbel-max decisions
 * drawn from `uniforms` (B,L,H,S,T,b float32, contiguous) or, when it is
 * NULL, from the counter RNG with `seed`.  Writes `weights` (softmax over
 * samples, float32) and the sampled leaves into the record.  Needs ta_pool
 * first.  Replaces sample_non_causal_paths_forward (treeattn_cuda.cpp:116;
 * kernel sample_non_causal_paths.cu:54-241) and the softmax at
 * _autograd.py:692,495-498. */
int ta_sample(const ta_problem* p, const void* q, const float* uniforms, uint64_t seed,
              float* weights, void* record, void* stream);

/* Groups every (query, distinct sampled leaf block) pair by leaf block (a
 * stable counting sort per batch*head) into the record.  Needs ta_sample
 * first.  Replaces the sampled-index bookkeeping the reference keeps in
 * torch tensors (_autograd.py:685-700) with a per-block bucket that both the
 * leaf forward and the atomic-free backward walk. */
int ta_bucket(const ta_problem* p, void* record, void* stream);

/* Leaf-block attention and sample combine: out = sum_s w_s softmax(q K_blk^T) V_blk,
 * MFMA tiles per leaf-block bucket.  Needs ta_bucket first.  Replaces
 * weighted_value_sum_forward (treeattn_cuda.cpp:91; weighted_value_sum.cu:8-47). */
int ta_leaf_forward(const ta_problem* p, const void* q, const void* k, const void* v,
                    void* out, void* record, void* workspace, void* stream);

/* Whole forward: ta_pool + ta_sample + ta_bucket + ta_leaf_forward.  Replaces
 * _StochasticNonCausalTreeAttention.forward (_autograd.py:645-704). */
int ta_forward(const ta_problem* p, const void* q, const void* k, const void* v,
               const float* uniforms, uint64_t seed, void* out, float* weights,
               void* record, void* workspace, void* stream);

/* ta_forward without the workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference.  The pair rows the
 * combine sums (ta_forward's workspace) live in a static device array of
 * TA_STATIC_SCRATCH_BYTES per GPU (allocated when the library is first used on
 * that device and held until the process ends); the leaf forward runs over
 * groups of (batch, head)s whose rows fit in it.  Outputs and record are
 * bit-identical to ta_forward's.  Problems whose one (batch, head) needs more
 * (L * num_samples * head_dim * element size bytes) get TA_ERR_UNSUPPORTED.
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (other streams, other threads) race and must be serialized by the
 * caller.  The stream must belong to the current device.  Allocates nothing. */
#define TA_STATIC_SCRATCH_BYTES ((int64_t)128 << 20)
int ta_forward_static(const ta_problem* p, const void* q, const void* k, const void* v,
                      const float* uniforms, uint64_t seed, void* out, float* weights, void* record,
                      void* stream);

/* Streaming forward of the deterministic mode for bfloat16 / float16 inputs:
 * out = W V with _deterministic_attention's weights (_tree_mha.py:286-318)
 * without materializing the (L, N) weights (memory O(L D)).  q and out
 * (batch, position, head) strides, v (batch, token, head), `knodes` the N-1
 * heap-ordered node keys in the input type with (batch, node, head) strides;
 * head dim 32/64/96/128, contiguous; other strides multiples of 8 elements.
 * N = 2^T with 64 <= N <= TA_DET_MAX_LEAVES.  Causal (leaves n <= l): `lse`
 * (B, H, L) float32, optional, receives each row's log-normalizer.  Replaces
 * _deterministic_attention's forward (_tree_mha.py:271-321) on the adapter's
 * path (baselines/treeattn_torch.py:55-90), which returns no weights. */
int ta_det_stream_forward(int dtype, const void* q, const int64_t* q_strides, const void* knodes,
                          const int64_t* k_strides, const void* v, const int64_t* v_strides, void* out,
                          const int64_t* o_strides, float* lse, int64_t B, int64_t L, int64_t H,
                          int64_t D, int64_t N, int causal, void* stream);

/* Its backward, streaming as well (no (L, N) buffer), in two parts:
 *  - here: `dq_sub` (B, H, L, D) float32, the gradient through the nodes of
 *    every 64-leaf subtree; `dknodes` (N-1, B, H, D) float32 rows of those
 *    nodes; `dv` (value strides, input type); `chunk_totals` (B, H, L, N/64)
 *    float32, each row's sum of dL/dlog w over each 64-leaf chunk;
 *  - by the caller: the N/64 - 1 top nodes are the deterministic mode on a
 *    coarse tree whose leaves are the chunks: X_top = q K_top^T, then
 *    ta_det_grad with W = chunk_totals, dW = 1, non-causal gives G_top;
 *    dq = dq_sub + G_top K_top, dknodes[top] = G_top^T q.
 * Causal needs `lse` (from ta_det_stream_forward) and `delta` (B, H, L) =
 * rowwise dout . out.  Replaces the autograd of _deterministic_attention
 * (_tree_mha.py:271-321) on the adapter's path. */
int ta_det_stream_backward(int dtype, const void* q, const int64_t* q_strides, const void* grad_out,
                           const int64_t* g_strides, const void* knodes, const int64_t* k_strides,
                           const void* v, const int64_t* v_strides, const float* lse, const float* delta,
                           float* dq_sub, float* chunk_totals, float* dknodes, void* dv,
                           const int64_t* dv_strides, int64_t B, int64_t L, int64_t H, int64_t D,
                           int64_t N, int causal, void* stream);

/* Packed path record of the reference (_autograd.py:68-90,179-216), the
 * stable on-device format of the sampled paths: per (position, batch, head,
 * sample) the root-to-leaf directions as a bit string, bit p (p = 0 at the
 * root) in byte p/8 at bit p%8, ta_path_bytes = ceil(log2(NL)/8) bytes,
 * layout (L, B, H, S, bytes) contiguous.  In a b-ary tree each level's child
 * digit takes log2(b) bits, high bit first, so the bit string is the leaf
 * block id most-significant bit first; for the reference's binary tree bit d
 * is the direction at depth d (heap walk node <- 2 node + 1 + dir).
 * `num_leaf_blocks` (NL) is a power of two; leaf ids are int32 in [0, NL)
 * with (batch, position, head, sample) element strides `leaf_strides[4]`
 * (the record's TA_REC_LEAVES array is (B, L, H, S) contiguous). */
int ta_path_bytes(int64_t num_leaf_blocks, int64_t* bytes);
int ta_pack_paths(const int32_t* leaf, const int64_t* leaf_strides, int64_t B, int64_t L, int64_t H,
                  int64_t S, int64_t num_leaf_blocks, uint8_t* packed, void* stream);
int ta_unpack_paths(const uint8_t* packed, int64_t B, int64_t L, int64_t H, int64_t S,
                    int64_t num_leaf_blocks, int32_t* leaf, const int64_t* leaf_strides, void* stream);

/* Path replay: ta_sample with every decision taken from `packed` (the layout
 * above, NL = N / leaf_block) instead of the Gumbel-max draw; log-probs,
 * weights and the record follow as in sampling, so replaying a forward's own
 * paths reproduces it bit for bit.  Non-causal problems only, like the
 * reference's replay.  Replaces _replay_non_causal_paths (_autograd.py:261-350)
 * and replay_non_causal_paths_forward (treeattn_cuda.cpp:142). */
int ta_replay(const ta_problem* p, const void* q, const uint8_t* packed, float* weights,
              void* record, void* stream);

/* Whole forward with replayed paths: ta_pool + ta_replay + ta_bucket + ta_leaf_forward. */
int ta_forward_replay(const ta_problem* p, const void* q, const void* k, const void* v,
                      const uint8_t* packed, void* out, float* weights, void* record,
                      void* workspace, void* stream);

/* Backward, leaf-block part: dv (complete), the leaf contribution to dk and
 * per-pair dq and dout.o into `workspace`.  For 16-bit inputs with b = 2 or
 * 4, leaf_block >= 2, T*b <= 32 and dense_cols = 0 it also takes the tree
 * gradient along every pair's sampled path (the pair's dq row then holds both
 * parts, and each leaf block's gradient of its path's child summaries goes to
 * `workspace`).  Replaces scatter_weighted_grad_v_forward
 * (treeattn_cuda.cpp:290) and the value side of prepare_non_causal_backward
 * (:176), without atomics. */
int ta_leaf_backward(const ta_problem* p, const void* q, const void* k, const void* v,
                     const void* grad_out, const void* record, void* dv, void* workspace, void* stream);

/* Backward, tree part (after ta_leaf_backward with the same workspace):
 * dq (complete) and dk (complete, including the summaries' adjoint).
 * Replaces accumulate_qk_non_causal_all_depths_prepared_inplace
 * (treeattn_cuda.cpp:211), the per-depth fallbacks (:321,:367) and the
 * autograd of the Haar keys (_treeattn_common.py:70-86). */
int ta_tree_backward(const ta_problem* p, const void* q, const float* weights, const void* record,
                     void* dq, void* dk, void* workspace, void* stream);

/* Whole backward from the forward's record: deterministic and atomic-free
 * dq, dk, dv (each fully overwritten).  Replaces
 * _StochasticNonCausalTreeAttention.backward (_autograd.py:706-860) with its
 * kernels prepare_non_causal_backward (treeattn_cuda.cpp:176),
 * scatter_weighted_grad_v_forward (:290),
 * accumulate_qk_non_causal_all_depths_prepared_inplace (:211) and the
 * per-depth fallbacks (:321,:367), plus the autograd of the Haar keys. */
int ta_backward(const ta_problem* p, const void* q, const void* k, const void* v,
                const void* grad_out, const float* weights, const void* record,
                void* dq, void* dk, void* dv, void* workspace, void* stream);

/* ---- deterministic (exact) mode, reference tree: binary, one token per leaf,
 * N = 2^T leaves, heap-ordered node keys (_tree_mha.py:271-321).  Rows are
 * (batch, head, query) rows laid out one after another; the dense products
 * around these calls (node logits X = Q K^T, out = W V and their gradients)
 * are plain batched GEMMs the caller runs.  N <= TA_DET_MAX_LEAVES. */
#define TA_DET_MAX_LEAVES 32768

/* W[r, n] = leaf-n weight of row r from its node logits X[r, 0..N-1)
 * (row strides ldx, ldw floats): prod of sigmoid(+-x) along n's path, or with
 * `causal` the softmax of the path log-probabilities over leaves n <= l, where
 * l = r % L is the row's query position.  Replaces the level loop and the
 * mask / softmax / exp of _deterministic_attention (_tree_mha.py:286-315). */
int ta_det_weights(const float* X, int64_t ldx, float* W, int64_t ldw, int64_t rows, int64_t L,
                   int64_t N, int causal, void* stream);

/* Node-logit gradient of every row, written over X: with dW = dout . v^T per
 * leaf, dlogw = W (dW - delta) (delta = sum_n W dW if causal, else 0) and
 * G[node] = sigmoid(-x) A_left - sigmoid(x) A_right, A = dlogw summed over a
 * child's leaves.  Replaces the autograd of _deterministic_attention
 * (_tree_mha.py:271-321) up to the GEMMs dq = G K, dK = G^T Q, dv = W^T dout. */
int ta_det_grad(float* XG, int64_t ldx, const float* W, const float* dW, int64_t ldw, int64_t rows,
                int64_t N, int causal, void* stream);

/* Heap-ordered Haar node keys of k (B, N, H, D with element strides
 * k_strides = {batch, position, head}) into out (N-1, B, H, D) float:
 * node m, p = m + 1, w = lowest set bit of p:
 * key = (mean k[p-w, p) - mean k[p, p+w)) / 2.  Replaces
 * haar_internal_node_keys (_treeattn_common.py:54-86) as read in heap order
 * by the op (_tree_mha.py:288-291).  With `workspace` (float scratch of
 * ta_haar_workspace_bytes, 16-byte aligned) the keys come from a block-sum
 * pyramid in O(N) work per (batch, head) and dim; with NULL, from per-node
 * window sums (O(N log N), no scratch). */
int ta_haar_workspace_bytes(int64_t B, int64_t H, int64_t D, int64_t N, int64_t* bytes);
int ta_haar_keys(int dtype, const void* k, const int64_t* k_strides, float* out, float* workspace,
                 int64_t B, int64_t H, int64_t D, int64_t N, void* stream);

/* dk (B, N, H, D, strides dk_strides, fully overwritten) = transpose of
 * ta_haar_keys applied to dkey (N-1, B, H, D) float.  Replaces the autograd of
 * haar_internal_node_keys (_treeattn_common.py:70-86). */
int ta_haar_keys_adjoint(int dtype, const float* dkey, void* dk, const int64_t* dk_strides, int64_t B,
                         int64_t H, int64_t D, int64_t N, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TREEATTN_AMD_H */
