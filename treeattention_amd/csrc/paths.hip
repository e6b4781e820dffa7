// The reference's packed path record (_autograd.py:68-90,179-216): per
// (position, batch, head, sample) the root-to-leaf directions as a bit
// string, bit p (p = 0 at the root) in byte p / 8 at bit p % 8,
// ceil(nbits / 8) bytes, layout (L, B, H, S, bytes).  In the b-ary tree each
// level's child digit contributes log2(b) bits, high bit first, so the bit
// string is the leaf block id written most-significant bit first; for the
// reference's binary tree bit d is the direction taken at depth d (the heap
// walk node <- 2 node + 1 + dir ends at leaf node - K).
//
// One thread per path: pack reads the leaf id (any strides) and writes its
// bytes; unpack is the inverse.
#include "launch.h"

namespace ta {

struct PathArgs {
  int64_t B, L, H, S;
  int64_t sb, sl, sh, ss;  // leaf-id strides (elements) of the (b, l, h, s) dims
  int nbits, nbytes;
};

__device__ __forceinline__ void path_coords(int64_t i, const PathArgs& a, int64_t& b, int64_t& l, int64_t& h,
                                            int64_t& s) {
  // i enumerates the packed layout (L, B, H, S)
  s = i % a.S;
  int64_t r = i / a.S;
  h = r % a.H;
  r /= a.H;
  b = r % a.B;
  l = r / a.B;
}

__global__ __launch_bounds__(256) void pack_paths_kernel(const int* __restrict__ leaf, uint8_t* __restrict__ packed,
                                                         PathArgs a, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int64_t b, l, h, s;
  path_coords(i, a, b, l, h, s);
  const uint32_t w = leaf_path_word((uint32_t)leaf[b * a.sb + l * a.sl + h * a.sh + s * a.ss], a.nbits);
  uint8_t* o = packed + i * a.nbytes;
  for (int k = 0; k < a.nbytes; ++k) o[k] = (uint8_t)(w >> (8 * k));
}

__global__ __launch_bounds__(256) void unpack_paths_kernel(const uint8_t* __restrict__ packed, int* __restrict__ leaf,
                                                           PathArgs a, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int64_t b, l, h, s;
  path_coords(i, a, b, l, h, s);
  leaf[b * a.sb + l * a.sl + h * a.sh + s * a.ss] = (int)path_leaf(packed + i * a.nbytes, a.nbits, a.nbytes);
}

static PathArgs path_args(int64_t B, int64_t L, int64_t H, int64_t S, const int64_t* st, int nbits) {
  PathArgs a;
  a.B = B;
  a.L = L;
  a.H = H;
  a.S = S;
  a.sb = st[0];
  a.sl = st[1];
  a.sh = st[2];
  a.ss = st[3];
  a.nbits = nbits;
  a.nbytes = (nbits + 7) / 8;
  return a;
}

hipError_t launch_pack_paths(const int* leaf, const int64_t* st, int64_t B, int64_t L, int64_t H, int64_t S,
                             int nbits, uint8_t* packed, hipStream_t stream) {
  const int64_t n = B * L * H * S;
  if (n == 0 || nbits == 0) return hipSuccess;
  hipLaunchKernelGGL(pack_paths_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, leaf, packed,
                     path_args(B, L, H, S, st, nbits), n);
  return hipGetLastError();
}

hipError_t launch_unpack_paths(const uint8_t* packed, int64_t B, int64_t L, int64_t H, int64_t S, int nbits,
                               int* leaf, const int64_t* st, hipStream_t stream) {
  const int64_t n = B * L * H * S;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(unpack_paths_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, packed, leaf,
                     path_args(B, L, H, S, st, nbits), n);
  return hipGetLastError();
}

}  // namespace ta
