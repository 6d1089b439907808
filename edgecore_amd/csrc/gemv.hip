// Decode / skinny GEMV kernels for gfx950 with fused prologues and epilogues.
//
//   out[m][n] = epilogue( dot( act[m][:], W[n][:] ) )       m < M (tiles of MT rows)
//
// Weights keep the reference layout [N][K] row-major (int8, fp16 or bf16).
// A row is read by LPR lanes of a wave with 16-byte non-temporal loads: one
// wave instruction covers 64/LPR rows x LPR*16 contiguous bytes.  A block of
// 256 threads (4 waves) owns a "row group" of 4*64/LPR output rows (2*64/LPR
// gate/up row pairs for SwiGLU) and walks the row groups grid-stride, so the
// prologue runs once per block and the first row group's weights are already
// in flight (prefetched into registers) while it runs.
//
// Prologues (activation side, computed redundantly by every block, which is
// cheaper than a separate launch at decode sizes):
//   PRO_I8    int8 rows + scales given (the gemm_int8 ABI)
//   PRO_F32   fp32 rows given (16-bit weights)
//   PRO_QUANT fp32 rows -> per-row int8 quantization (src/gpt2.c:446-461)
//   PRO_RMS   RMSNorm (src/gpt2.c:592-604), then quantize (int8) or keep fp32
//   PRO_LN    LayerNorm (src/gpt2.c:398-414), then quantize (int8) or keep fp32
// Norms accumulate in double exactly like the reference formula; only the
// order of the double additions differs (a fixed tree).
//
// int8 dots use v_dot4_i32_i8 into an exact int32, so every summation order
// gives the reference's value and the epilogue bias + ((float)dot*as)*bs is
// bit-exact.  16-bit weights are widened to fp32 and accumulated with FMA.
#include "ec_device.h"
#include "ec_kernels.h"

#include <float.h>

namespace ec {

constexpr int kThreads = 256;

// orderable 64-bit key: larger key = larger value, ties -> lower index.
// -0 is folded onto +0 (the reference compares with >, so they tie).
__device__ __forceinline__ unsigned long long amax_key(float v, int n) {
  v = v + 0.0f;
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)n);
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    unsigned long long w = __shfl_xor(v, o, kWave);
    v = w > v ? w : v;
  }
  return v;
}

// ---------------------------------------------------------------------------
// prologue: MT activation rows -> LDS (int8 + scale, or fp32)
// ---------------------------------------------------------------------------

template <int PRO, bool Q8, int JMAX>
__device__ __forceinline__ void prologue(const GemvArgs &a, int m0, int mc, unsigned char *lds,
                                         int Kp, double *redd, float *redf) {
  const int t = threadIdx.x;
  int8_t *xq = reinterpret_cast<int8_t *>(lds);
  float *xs = reinterpret_cast<float *>(lds + (size_t)MT_ROWS_MAX * 0);  // placeholder, replaced below
  (void)xs;
  (void)xq;
}

}  // namespace ec
