// Host-side plan and kernel launchers shared by the C ABI (capi.cpp).
#pragma once

#include "common.h"

namespace ta {

// A problem with more samples than one launch takes (kMaxSamples) runs as
// chunks of samples, each a plan of its own; these float accumulators in the
// caller's record / workspace carry the sums across the chunks (all null for
// a single-chunk problem).  The first chunk writes them, later chunks add in
// chunk order (deterministic), and the last chunk runs the key adjoint.
struct ChunkAcc {
  float* out32;       // (B, L, H, D) forward output
  float* dq32;        // (B, L, H, D)
  float* dv32;        // (B, N, H, D)
  float* dk_leaf;     // (B, N, H, D) leaf-attention part of dk
  float* dsum;        // (BH, NS, D) summary gradient
  const float* mean;  // (B, L, H) dout . out over every sample of the query
  int first, last;
};

// Everything derived from a ta_problem that the launchers need.
struct Plan {
  ta_problem p;
  Geo geo;
  int64_t B, L, N, H, D, S, BH;  // L queries, N leaf tokens
  int esize;        // bytes per element of q/k/v
  int qc;           // queries per bucketing chunk
  int nchunk;       // bucketing chunks per (batch, head)
  int npiece;       // leaf-forward pieces per (batch, head), upper bound
  int nseg;         // scan segments of the bucket histogram per (batch, head)
  int64_t Lp;       // L rounded up to a multiple of kQueryTile
  int qsplit;       // query splits of the summary-gradient product
  int sample_dense; // the sampler's level tiles cover depths < sample_dense; deeper levels are sparse
  int tree_dense;   // the backward's dense G tiles cover depths < tree_dense; deeper ones run in bands
  int bucket_sort;  // many leaf blocks: bucketing by a radix sort of (batch * head, leaf block) keys
  int leaf_path;    // > 0 (one-token leaves): the tree gradient along the paths per subtree of
                   // 2^leaf_path leaves (leaf_path1.hip) instead of dense levels and bands
  int path_rows;    // > 0: the leaf backward adds the tree gradient along each pair's path (T*b rows,
                   // padded to 16 or 32); the tree backward only sums rows and blocks
  int64_t s0, s_total;  // this plan's samples are s0 .. s0 + S - 1 of s_total (uniform / path indices)
  ChunkAcc acc;
  RecordLayout rec;
  FwdWorkspaceLayout fws;
  BwdWorkspaceLayout bws;
};

// A problem's chunks of samples: num_samples <= kMaxSamples is one chunk
// whose plan is the problem's own.  With more samples chunk g takes samples
// s0_g .. s0_g + S_g - 1 (sizes within one of each other), has a record of
// its own inside the caller's record, and reuses one forward / backward
// workspace after the other; the record also holds every sample's leaf block
// and the float forward output, the backward workspace the accumulators.
constexpr int kMaxChunks = 16;  // num_samples <= kMaxChunks * kMaxSamples
struct Chunks {
  int n;
  Plan P[kMaxChunks];
  int64_t rec_off[kMaxChunks];  // chunk g's record
  int64_t rec_leaf;             // int (B, L, H, S): every sample's leaf block (n > 1)
  int64_t rec_out32;            // float (B, L, H, D): the forward output before rounding (n > 1)
  int64_t rec_total, fws_total;
  int64_t bws_dq32, bws_dv32, bws_dkl, bws_dsum, bws_mean, bws_chunk, bws_total;
};

// capi.cpp: plan builder and the calling thread's error message
// TA_OK or an error code (message set); chunk: a chunk of a problem with many
// samples (whose float output lives in the problem's record, not the chunk's)
int make_plan(const ta_problem* p, Plan* P, bool chunk = false);
int make_chunks(const ta_problem* p, Chunks* C);
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int ok();  // clears the message, returns TA_OK
const char* last_error();

// pool.hip
hipError_t launch_pool(const Plan& P, const void* k, char* rec, hipStream_t st);
hipError_t launch_fill_uniforms(uint64_t seed, int64_t n, float* out, hipStream_t st);
// sample.hip
// paths (optional): packed path bits (L, B, H, S, bytes) whose directions
// replace the Gumbel-max decisions (non-causal problems)
hipError_t launch_sample(const Plan& P, const void* q, const float* U, uint64_t seed,
                         float* weights, char* rec, hipStream_t st, const uint8_t* paths = nullptr);
// sample_replay.hip
hipError_t launch_sample_replay(const Plan& P, const void* q, float* weights, char* rec, hipStream_t st,
                                const uint8_t* paths);
// paths.hip (packed path bits; leaf ids with (b, l, h, s) strides st)
hipError_t launch_pack_paths(const int* leaf, const int64_t* st, int64_t B, int64_t L, int64_t H, int64_t S,
                             int nbits, uint8_t* packed, hipStream_t stream);
hipError_t launch_unpack_paths(const uint8_t* packed, int64_t B, int64_t L, int64_t H, int64_t S, int nbits,
                               int* leaf, const int64_t* st, hipStream_t stream);
// sample_ref.hip (reference causal mode)
hipError_t launch_ref_sample(const Plan& P, const void* q, const float* U, uint64_t seed,
                             float* weights, char* rec, hipStream_t st);
// bucket.hip
hipError_t launch_bucket(const Plan& P, char* rec, hipStream_t st);
// leaf_fwd.hip
hipError_t launch_leaf_fwd(const Plan& P, const void* q, const void* k, const void* v,
                           void* out, char* rec, char* ws, hipStream_t st);
// The leaf forward of the (batch, head)s bh0 .. bh0 + nbh - 1 only, with their
// partial rows in `partial` ((nbh, L, S, D) elements of the input type).
hipError_t launch_leaf_fwd_group(const Plan& P, const void* q, const void* k, const void* v, void* out, char* rec,
                                 void* partial, int bh0, int nbh, hipStream_t st);
// leaf_bwd.hip
hipError_t launch_leaf_bwd(const Plan& P, const void* q, const void* k, const void* v,
                           const void* g, const char* rec, void* dv, char* ws, hipStream_t st);
// tree_bwd.hip
hipError_t launch_tree_bwd(const Plan& P, const void* q, const float* weights, const char* rec,
                           void* dq, void* dk, char* ws, hipStream_t st);

// det.hip (deterministic mode)
hipError_t launch_det_weights(const float* X, int64_t ldx, float* W, int64_t ldw, int64_t rows, int L, int N, int T,
                              int causal, hipStream_t st);
hipError_t launch_det_grad(float* XG, int64_t ldx, const float* W, const float* dW, int64_t ldw, int64_t rows, int N,
                           int T, int causal, hipStream_t st);
hipError_t launch_haar_keys(int dtype, const void* k, const int64_t* ks, float* out, float* segsum, int B, int H,
                            int D, int N, hipStream_t st);
int64_t haar_workspace_floats(int B, int H, int D, int N);
hipError_t launch_haar_keys_adjoint(int dtype, const float* dkey, void* dk, const int64_t* ks, int B, int H, int D,
                                    int N, int T, hipStream_t st);

// det_stream.hip (deterministic mode, streaming forward for 16-bit inputs)
hipError_t launch_det_stream_fwd(int dtype, const void* q, const int64_t* qs, const void* kn, const int64_t* ks,
                                 const void* v, const int64_t* vs, void* out, const int64_t* os, float* lse, int B,
                                 int L, int H, int D, int T, int causal, hipStream_t st);

// det_stream_bwd.hip (its backward: dq and node-key gradients of the 64-leaf subtrees, dv)
hipError_t launch_det_stream_bwd(int dtype, const void* q, const int64_t* qs, const void* gout, const int64_t* gs,
                                 const void* kn, const int64_t* ks, const void* v, const int64_t* vs, const float* lse,
                                 const float* delta, float* dq, float* achunk, float* dkn, void* dv,
                                 const int64_t* dvs, int B, int L, int H, int D, int T, int causal, hipStream_t st);

// chunks.hip (more samples than one chunk): after every chunk's sampler, the
// per-query log-normalizers give each chunk's share alpha_g = exp(lse_g - lse)
// of the query; the chunk's weights (w + s0_g, caller strides) and the summed
// weights of its record are scaled by it; every chunk's leaf blocks are copied
// into leaf_all (B, L, H, S).
struct ChunkRecs {
  int n;
  int S[kMaxChunks], s0[kMaxChunks];
  const float* lse[kMaxChunks];  // pieces of chunk g's record
  float* slot_weight[kMaxChunks];
  const int* slot_count[kMaxChunks];
  const int* leaf[kMaxChunks];
};
hipError_t launch_chunk_merge(const Plan& P, const ChunkRecs& R, float* weights, int* leaf_all, hipStream_t st);
// mean[b,l,h] = dout . out32 over the head dim
// out: (B, L, H, D) rows of the forward output, float or (out_e) the input type
hipError_t launch_chunk_mean(const Plan& P, const void* g, const void* out, bool out_e, float* mean, hipStream_t st);
// dst (E, strides st3 (batch, row, head)) = src (float (B, R, H, D) contiguous)
hipError_t launch_cast_rows(int dtype, const float* src, void* dst, const int64_t* st3, int64_t B, int64_t R,
                            int64_t H, int64_t D, hipStream_t st);

// leaf_gather.hip (leaf_block 1: the leaf stage is a value gather)
hipError_t launch_gather_fwd(const Plan& P, const void* v, void* out, const char* rec, int bh0, int nbh,
                             hipStream_t st);
hipError_t launch_gather_bwd(const Plan& P, const void* v, const void* g, void* dv, const char* rec, char* ws,
                             hipStream_t st);

// Leaf-kernel shared-memory need (bytes) for the chosen tile, or -1 if no
// variant fits in 160 KiB.
int leaf_fwd_smem(const Plan& P);
int ref_sample_smem(const Plan& P);
int leaf_bwd_smem(const Plan& P);
// leaf_path1.hip
int leaf_path1_depth(int T);
int leaf_path1_top_rows();
int leaf_path1_smem(int D);
hipError_t launch_leaf_path1(const Plan& P, const void* q, const char* rec, char* ws, float* dsum, int first,
                             hipStream_t st);

inline int padded_keys(int LB) { return LB <= 32 ? 32 : (LB <= 64 ? 64 : 128); }

}  // namespace ta
