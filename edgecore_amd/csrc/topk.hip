// Device top-k of logit rows for sampled decoding (the selection of
// sample_token, src/runtime_main.c:220-226, and what it reads): per row the
// top_k + 1 largest logits, value descending and index ascending among equal
// values, plus a status that tells whether they determine sample_token's
// choice (no NaN in the row, and the top_k-th and (top_k+1)-th values differ).
//
// Keys: an order-preserving 32-bit image of the float (sign bit flipped for
// positives, all bits for negatives) above the inverted index, so that one
// 64-bit comparison orders by value and then by smaller index.  -0 and +0
// get different keys; the status compares the boundary values as floats, so
// a -0/+0 pair at the boundary counts as a tie.
//
//   topk_chunk_kernel: a block of 512 threads sorts a chunk of 4096 logits
//     (bitonic, in LDS) and keeps its top n = top_k + 1 keys and a NaN flag;
//   topk_merge_kernel: one block of 1024 threads per row sorts the chunks'
//     candidates (at most 16384 keys) and writes the row's top n and status.
#include "ec_device.h"
#include "ec_kernels.h"

namespace ec {

namespace {

constexpr int kChunk = 4096;

__device__ __forceinline__ uint32_t fkey(float v) {
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float fkey_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}

// bitonic sort of S (a power of two) keys in LDS into descending order
template <int NT>
__device__ void sort_desc(unsigned long long *s, int S) {
  for (int k = 2; k <= S; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < S; i += NT) {
        const int l = i ^ j;
        if (l > i) {
          const unsigned long long a = s[i], b = s[l];
          const bool down = (i & k) == 0;  // this run descending
          if (down ? a < b : a > b) {
            s[i] = b;
            s[l] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

__global__ __launch_bounds__(512) void topk_chunk_kernel(const float *L, int ld, int V, int n,
                                                         unsigned long long *cand, unsigned char *nan_flag) {
  __shared__ unsigned long long s[kChunk];
  __shared__ int has_nan;
  const int row = blockIdx.y, c0 = blockIdx.x * kChunk;
  const float *l = L + (size_t)row * ld;
  if (threadIdx.x == 0) has_nan = 0;
  __syncthreads();
  bool nan_here = false;
  for (int i = threadIdx.x; i < kChunk; i += 512) {
    const int v = c0 + i;
    unsigned long long key = 0;  // below every key of a number
    if (v < V) {
      const float x = l[v];
      nan_here |= x != x;
      key = ((unsigned long long)fkey(x) << 32) | (0xFFFFFFFFu - (uint32_t)v);
    }
    s[i] = key;
  }
  if (nan_here) has_nan = 1;
  __syncthreads();
  sort_desc<512>(s, kChunk);
  unsigned long long *out = cand + ((size_t)row * gridDim.x + blockIdx.x) * n;
  for (int i = threadIdx.x; i < n; i += 512) out[i] = s[i];
  if (threadIdx.x == 0) nan_flag[(size_t)row * gridDim.x + blockIdx.x] = (unsigned char)has_nan;
}

__global__ __launch_bounds__(1024) void topk_merge_kernel(const unsigned long long *cand,
                                                          const unsigned char *nan_flag, int nb, int n,
                                                          int top_k, int S, float *vals, int *idx,
                                                          int *status) {
  extern __shared__ unsigned long long s[];  // S keys
  __shared__ int has_nan;
  const int row = blockIdx.x, tot = nb * n;
  const unsigned long long *c = cand + (size_t)row * tot;
  if (threadIdx.x == 0) has_nan = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < S; i += 1024) s[i] = i < tot ? c[i] : 0ull;
  for (int b = threadIdx.x; b < nb; b += 1024)
    if (nan_flag[(size_t)row * nb + b]) has_nan = 1;
  __syncthreads();
  sort_desc<1024>(s, S);
  for (int i = threadIdx.x; i < n; i += 1024) {
    vals[(size_t)row * n + i] = fkey_value((uint32_t)(s[i] >> 32));
    idx[(size_t)row * n + i] = (int)(0xFFFFFFFFu - (uint32_t)s[i]);
  }
  if (threadIdx.x == 0) {
    const float a = fkey_value((uint32_t)(s[top_k - 1] >> 32)), b = fkey_value((uint32_t)(s[top_k] >> 32));
    status[row] = (has_nan || a == b) ? 1 : 0;
  }
}

int merge_size(int nb, int n) {
  int S = 1;
  while (S < nb * n) S <<= 1;
  return S;
}

}  // namespace

int topk_chunks(int V) { return (V + kChunk - 1) / kChunk; }

bool topk_ok(int V, int top_k) {
  return top_k > 0 && top_k < V && top_k <= kTopkMax && merge_size(topk_chunks(V), top_k + 1) <= 16384;
}

hipError_t topk_select(const float *L, int rows, int V, int ld, int top_k, unsigned long long *cand,
                       unsigned char *nan_flag, hipStream_t st) {
  if (!topk_ok(V, top_k) || rows < 1) return hipErrorInvalidValue;
  klaunch(topk_chunk_kernel, dim3(topk_chunks(V), rows), dim3(512), 0, st, L, ld, V, top_k + 1, cand, nan_flag);
  return hipGetLastError();
}

hipError_t topk_merge(const unsigned long long *cand, const unsigned char *nan_flag, int rows, int V, int top_k,
                      float *vals, int *idx, int *status, hipStream_t st) {
  if (!topk_ok(V, top_k) || rows < 1) return hipErrorInvalidValue;
  const int nb = topk_chunks(V), n = top_k + 1, S = merge_size(nb, n);
  klaunch(topk_merge_kernel, dim3(rows), dim3(1024), (uint32_t)(S * sizeof(unsigned long long)), st, cand,
          nan_flag, nb, n, top_k, S, vals, idx, status);
  return hipGetLastError();
}

}  // namespace ec
