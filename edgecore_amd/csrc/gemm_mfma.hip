// GEMMs on the gfx950 matrix cores for the linears of a prefill and of
// batched decode (M >= kGemmMinM rows).
//
// int8 weights (src/kernels.c:153-168, gemm_int8, with the epilogues
// src/gpt2.c applies after it: residual add :782-784, SwiGLU :788-791, GELU
// :568):
//
//   C[m][n] = epi( bias[n] + ((float)sum_k A[m][k]*B[n][k] * as[m]) * bs[n] )
//
// The int32 dot is exact whatever the summation order, so
// v_mfma_i32_16x16x64_i8 reproduces the reference's dot bit for bit; the fp32
// epilogue is the same device code as the decode GEMV's (i8_epilogue, silu,
// gelu_new), so a row gives the same floats through either kernel.
//
// 16-bit weights (src/kernels.c:129-151, gemm_fp16_fp32 / gemm_bf16_fp32:
// fp32 activations times fp16 or bf16 weights, fp32 sums).  The matrix cores
// multiply 16-bit operands, so split_rows first writes every fp32 activation
// row as a sum of 16-bit parts that the products see exactly:
//   fp16 weights: x = 2^e (h + l), h = fp16(x 2^-e), l = fp16(x 2^-e - h),
//                 with e = ilogb(max_k |x|) - 14 per row, so that h stays in
//                 fp16 range and h + l carries 22 significant bits;
//   bf16 weights: x = h + m + l, three bf16 parts (24 bits, fp32 range).
// Each product of a 16-bit weight and a 16-bit part is exact in fp32 and the
// matrix core sums in fp32, so C[m][n] = 2^e * sum_parts sum_k B[n][k] * part
// differs from the reference's sequential fp32 dot only by fp32 rounding of
// the sums (and by the < 2^-22 relative residue of the split) -- the same
// class of difference as the vector GEMV's reordered fp32 sums.
//
// Tiling: a block of 256 threads (4 waves, 2 x 2) computes a BM x 128 tile of
// C (for SwiGLU: BM x 64 outputs, each from a gate row and an up row).  K runs
// in stages of 128 bytes (128 int8 or 64 16-bit elements) through two LDS
// buffers; each thread holds the next stage's 16-byte chunks in registers
// while the waves multiply the current one.  Rows of the LDS tiles are 144
// bytes apart, so the 16-byte fragment reads of 8 consecutive lanes (16 rows,
// same k) fall on distinct banks.  The activation tile holds NP parts (1 for
// int8, 2 for fp16, 3 for bf16), part-major.
//
// MFMA lane layout (16x16x64 i8 and 16x16x32 f16 / bf16, checked on the
// device): lane l supplies row l % 16 of A (column l % 16 of B) with the 16
// bytes at byte offset 16*(l/16) of the 64-byte k-slice, and receives
// D[4*(l/16) + r][l % 16] in accumulator register r.
#include "ec_device.h"
#include "ec_kernels.h"

namespace ec {

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr int kBK = 128;            // K bytes per LDS stage
constexpr int kPitch = kBK + 16;    // LDS row pitch in bytes
constexpr int kBN = 128;            // B rows per block tile

// operand kinds: int8 x int8 -> int32, fp16 x fp16 -> fp32, bf16 x bf16 -> fp32
enum { OP_I8 = 0, OP_F16 = 1, OP_BF16 = 2 };

template <int OP>
struct MfmaOp;
template <>
struct MfmaOp<OP_I8> {
  static constexpr int NP = 1, EB = 1;  // activation parts, bytes per element
  using Acc = v4i;
  static __device__ __forceinline__ Acc mma(v4i a, v4i b, Acc c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
  }
};
template <>
struct MfmaOp<OP_F16> {
  static constexpr int NP = 2, EB = 2;
  using Acc = v4f;
  static __device__ __forceinline__ Acc mma(v4i a, v4i b, Acc c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0, 0);
  }
};
template <>
struct MfmaOp<OP_BF16> {
  static constexpr int NP = 3, EB = 2;
  using Acc = v4f;
  static __device__ __forceinline__ Acc mma(v4i a, v4i b, Acc c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c, 0, 0,
                                                   0);
  }
};

// NB stage buffers (2, or up to 4 in the direct-to-LDS form); the
// direct-to-LDS form (DL) has unpadded rows
template <int OP, int BM, bool DL, int NB = 2>
constexpr size_t gemm_lds_bytes() {
  return (size_t)NB * (MfmaOp<OP>::NP * BM + kBN) * (DL ? kBK : kPitch);
}

// Split K of the tiled kernel: gridDim.y blocks share a tile, each taking a
// contiguous range of K stages; each stores its 32-bit accumulators to
// gm_part, and the tile's last block to arrive (a counter per tile, reset by
// that block, so every launch finds it at zero) adds the gridDim.y partial
// tiles in y order and applies the epilogue.  For int8 the sums are exact;
// for 16-bit weights the fp32 sums take a fixed order, the same class of
// rounding as the one-block tile.  One workspace per device: launches that
// use it must not overlap (the forward issues its linears on one stream).
constexpr int kGmMaxTiles = 1024;         // tiles of a split launch
constexpr int kGmPartInts = 1024 * 1024;  // 32-bit partial tiles of a split launch
__device__ int gm_part[kGmPartInts];
__device__ unsigned gm_cnt[kGmMaxTiles];

// A: [M * NP][lda] elements (row m's part p at row m * NP + p), as: per-row
// scale (int8 quantization scale, or the split's 2^e; 1 for bf16)
template <int OP, int BM, int EPI, bool DL, int NB = 2, bool SPLIT = false>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(GemvArgs a) {
  using Op = MfmaOp<OP>;
  using Acc = typename Op::Acc;
  constexpr int NP = Op::NP;
  constexpr bool I8 = OP == OP_I8;
  constexpr bool SWI = EPI == EPI_SWIGLU;
  constexpr bool RES = EPI == EPI_RESID || EPI == EPI_BIAS_RESID;
  constexpr bool GELU = EPI == EPI_GELU || EPI == EPI_BIAS_GELU;
  constexpr int WM = BM / 2, WN = kBN / 2;   // wave tile
  constexpr int TI = WM / 16, TJ = WN / 16;  // 16 x 16 MFMA tiles per wave
  constexpr int CPR = kBK / 16;              // 16-byte chunks per tile row and stage
  constexpr int ACH = NP * BM * CPR / 256;   // A chunks per thread and stage
  constexpr int BCH = kBN * CPR / 256;       // B chunks per thread and stage
  constexpr int NOUT = SWI ? kBN / 2 : kBN;  // output columns per block
  static_assert(ACH >= 1 && BCH >= 1 && TJ % 2 == 0 && NP * BM * CPR % 256 == 0, "tile shape");

  extern __shared__ __attribute__((aligned(16))) int8_t lds[];
  int8_t *la = lds;                            // [2][NP][BM][kPitch]
  int8_t *lb = lds + 2 * NP * BM * kPitch;     // [2][kBN][kPitch]
  __shared__ uint64_t etab[SWI ? 32 : 1];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 15, lq = lane >> 4;
  const int M = a.M, K = a.K, N = a.N;
  const int KB = K * Op::EB;  // bytes of a weight row and of an activation part row
  const size_t ldab = (size_t)a.lda * Op::EB;
  // XCD-aware tile order: block b runs on XCD b % 8; XCD x takes tiles
  // [x * per, (x + 1) * per) of the weight-row-major order, i.e. a contiguous
  // share of the weight rows with every row tile of A, so its L2 holds both
  const int nM = (M + BM - 1) / BM, nN = (N + NOUT - 1) / NOUT, T = nM * nN, per = (T + 7) / 8;
  const int tl = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if (tl >= T) return;
  const int m0 = (tl % nM) * BM, n0 = (tl / nM) * NOUT;
  if constexpr (SWI) {
    if (t < 32) etab[t] = ec_exp2_32[t];
  }

  // epilogue operands, loaded before the K loop so that their latency hides
  // behind it: the row scales of this lane's rows, the weight scales / bias
  // of its columns and, for a residual, the old output values.  Indices are
  // clamped into the matrix and absent vectors read a stand-in (the weight
  // rows); the values are selected at use.
  constexpr int JO = SWI ? TJ / 2 : TJ;  // output column tiles
  const int lrow0 = m0 + wm * WM + 4 * lq, lcol0 = n0 + (SWI ? wn * (kBN / 4) : wn * WN) + lr;
  float e_as[TI][4], e_bs[JO], e_bv[JO], e_bs2[JO];
  float e_old[RES ? TI : 1][RES ? JO : 1][4];
  {
    const float *stand = (const float *)a.W;  // N*K >= 4N bytes: valid for every column index
    const float *wsp = a.ws ? a.ws : stand, *bvp = a.bias ? a.bias : stand;
    const float *ws2p = (SWI && a.ws2) ? a.ws2 : stand;
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) e_as[i][r] = a.as[min(lrow0 + 16 * i + r, M - 1)];
#pragma unroll
    for (int j = 0; j < JO; j++) {
      const int n = min(lcol0 + 16 * j, N - 1);
      e_bs[j] = wsp[n];
      e_bv[j] = bvp[n];
      e_bs2[j] = ws2p[n];
    }
    if constexpr (RES) {
#pragma unroll
      for (int i = 0; i < TI; i++)
#pragma unroll
        for (int j = 0; j < JO; j++)
#pragma unroll
          for (int r = 0; r < 4; r++)
            e_old[i][j][r] = a.out[(size_t)min(lrow0 + 16 * i + r, M - 1) * a.ldo + min(lcol0 + 16 * j, N - 1)];
    }
  }

  // global chunk sources of this thread: tile row, 16-byte column, row base.
  // A chunk c covers tile row r = c / CPR of the part-major tile: part r / BM
  // of activation row m0 + r % BM.
  const int8_t *arow[ACH];
  const int8_t *brow[BCH];
  int acol[ACH], bcol[BCH], aoff[ACH], boff[BCH];
  const int8_t *A = (const int8_t *)a.A;
#pragma unroll
  for (int j = 0; j < ACH; j++) {
    const int c = t + 256 * j, r = c / CPR;
    const int p = r / BM, mr = r % BM;
    acol[j] = c % CPR;
    arow[j] = A + ((size_t)min(m0 + mr, M - 1) * NP + p) * ldab;
    aoff[j] = r * kPitch + 16 * acol[j];
  }
#pragma unroll
  for (int j = 0; j < BCH; j++) {
    const int c = t + 256 * j, r = c / CPR;
    bcol[j] = c % CPR;
    const int8_t *W = (const int8_t *)a.W;
    int n = n0 + r;
    if (SWI && r >= kBN / 2) {
      W = (const int8_t *)a.W2;
      n = n0 + r - kBN / 2;
    }
    brow[j] = W + (size_t)min(n, N - 1) * KB;
    boff[j] = r * kPitch + 16 * bcol[j];
  }

  // chunks past the row (a last stage shorter than kBK) are loaded clamped and
  // zeroed when stored to LDS, so that nothing waits on the loads before the
  // multiplies of the current stage
  v4i ra[ACH], rb[BCH];
  int kl = 0;  // byte offset of the stage held in ra / rb
  auto load = [&](int k0) {
    kl = k0;
#pragma unroll
    for (int j = 0; j < ACH; j++)
      ra[j] = *reinterpret_cast<const v4i *>(arow[j] + min(k0 + 16 * acol[j], KB - 16));
#pragma unroll
    for (int j = 0; j < BCH; j++)
      rb[j] = *reinterpret_cast<const v4i *>(brow[j] + min(k0 + 16 * bcol[j], KB - 16));
  };
  auto store = [&](int buf) {
    const v4i z = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < ACH; j++)
      *reinterpret_cast<v4i *>(la + buf * NP * BM * kPitch + aoff[j]) = kl + 16 * acol[j] < KB ? ra[j] : z;
#pragma unroll
    for (int j = 0; j < BCH; j++)
      *reinterpret_cast<v4i *>(lb + buf * kBN * kPitch + boff[j]) = kl + 16 * bcol[j] < KB ? rb[j] : z;
  };

  // B tile rows of this wave's column tiles: plain, or gate (j < TJ/2) and up
  int bt[TJ];
#pragma unroll
  for (int j = 0; j < TJ; j++) {
    if constexpr (SWI) {
      const int jj = j % (TJ / 2);
      bt[j] = (j < TJ / 2 ? 0 : kBN / 2) + wn * (kBN / 4) + 16 * jj;
    } else {
      bt[j] = wn * WN + 16 * j;
    }
  }

  Acc acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; i++)
#pragma unroll
    for (int j = 0; j < TJ; j++) acc[i][j] = Acc{0, 0, 0, 0};

  // this block's K stages: [sb, sb + ns) of the row's, all of them unless split
  const int ns_all = (KB + kBK - 1) / kBK, kper = (ns_all + (int)gridDim.y - 1) / (int)gridDim.y;
  const int sb = (int)blockIdx.y * kper, ns = min(ns_all - sb, kper);
  const int kb0 = sb * kBK;
  if constexpr (!DL) {
    load(kb0);
    store(0);
    __syncthreads();
    for (int s = 0; s < ns; s++) {
      const int buf = s & 1;
      if (s + 1 < ns) load(kb0 + (s + 1) * kBK);
      const int8_t *ta = la + buf * NP * BM * kPitch + (wm * WM + lr) * kPitch + 16 * lq;
      const int8_t *tb = lb + buf * kBN * kPitch + lr * kPitch + 16 * lq;
  #pragma unroll
      for (int kk = 0; kk < kBK / 64; kk++) {
        v4i fa[NP][TI], fb[TJ];
  #pragma unroll
        for (int p = 0; p < NP; p++)
  #pragma unroll
          for (int i = 0; i < TI; i++)
            fa[p][i] = *reinterpret_cast<const v4i *>(ta + (p * BM + 16 * i) * kPitch + 64 * kk);
  #pragma unroll
        for (int j = 0; j < TJ; j++) fb[j] = *reinterpret_cast<const v4i *>(tb + bt[j] * kPitch + 64 * kk);
  #pragma unroll
        for (int p = 0; p < NP; p++)
  #pragma unroll
          for (int i = 0; i < TI; i++)
  #pragma unroll
            for (int j = 0; j < TJ; j++) acc[i][j] = Op::mma(fa[p][i], fb[j], acc[i][j]);
      }
      if (s + 1 < ns) store(buf ^ 1);
      __syncthreads();
    }
  } else {
    // Both tiles loaded straight into LDS (global_load_lds_dwordx4: lane l's
    // 16 bytes land 16 l bytes after the wave's base), rows of kBK bytes with
    // no padding; chunk c of row r sits at chunk c ^ (r & 7) of the row, so
    // that the 16-byte fragment reads of 8 consecutive rows hit distinct
    // banks.  A wave instruction fills 8 rows: lane l takes row 8 u + l / 8
    // and stores the row's chunk (l & 7) ^ (l / 8) at position l & 7.  Rows
    // are K-complete (the launcher takes this path when K bytes are a
    // multiple of kBK), so no chunk is past the row.
    constexpr int RT = NP * BM + kBN;  // tile rows per stage
    constexpr int UPW = RT / 32;       // 8-row load instructions per wave and stage
    static_assert(RT % 32 == 0, "tile rows");
    typedef __attribute__((address_space(1))) const void gvoid;
    typedef __attribute__((address_space(3))) void lvoid;
    const int lrow = lane >> 3, lchk = (lane & 7) ^ lrow;
    const int8_t *src[UPW];
#pragma unroll
    for (int u = 0; u < UPW; u++) {
      const int r = 8 * (wave * UPW + u) + lrow;  // tile row
      if (r < NP * BM) {
        const int p = r / BM, mr = r % BM;
        src[u] = A + ((size_t)min(m0 + mr, M - 1) * NP + p) * ldab + 16 * lchk;
      } else {
        const int rb = r - NP * BM;
        const int8_t *W = (const int8_t *)a.W;
        int n = n0 + rb;
        if (SWI && rb >= kBN / 2) {
          W = (const int8_t *)a.W2;
          n = n0 + rb - kBN / 2;
        }
        src[u] = W + (size_t)min(n, N - 1) * KB + 16 * lchk;
      }
    }
    auto dload = [&](int k0, int buf) {
      int8_t *base = lds + (size_t)buf * RT * kBK + (size_t)wave * UPW * 8 * kBK;
#pragma unroll
      for (int u = 0; u < UPW; u++)
        __builtin_amdgcn_global_load_lds((gvoid *)(src[u] + k0), (lvoid *)(base + u * 8 * kBK), 16, 0, 0);
    };
    const int sw = lr & 7;  // fragment rows are 16-aligned: row & 7 == lr & 7
    // NB stage buffers, NB - 1 stages in flight: stage s is waited for (each
    // wave its own loads -- the loads complete in order, so the NB - 2 later
    // stages' UPW instructions each may stay outstanding -- then the
    // barrier) before stage s + NB - 1 is loaded into the buffer that stage
    // s - 1 used, whose reads completed before the barrier.  The barrier is
    // bare: __syncthreads() adds a fence whose waits come out no better.
    // (Few tiles per CU wait on each stage's load latency: the C2 prefill
    // linears with NB 2 took ~1 us per stage.)
#pragma unroll
    for (int p = 0; p < NB - 1; p++)
      if (p < ns) dload(kb0 + p * kBK, p);
    for (int s = 0; s < ns; s++) {
      if (NB > 2 && s + NB - 2 < ns) asm volatile("s_waitcnt vmcnt(%0)" ::"i"((NB - 2) * UPW) : "memory");
      else __builtin_amdgcn_s_waitcnt(0);
      asm volatile("s_barrier" ::: "memory");
      if (s + NB - 1 < ns) dload(kb0 + (s + NB - 1) * kBK, (s + NB - 1) % NB);
      const int buf = s % NB;
      const int8_t *ta = lds + (size_t)buf * RT * kBK + (size_t)(wm * WM + lr) * kBK;
      const int8_t *tb = lds + (size_t)buf * RT * kBK + (size_t)(NP * BM + lr) * kBK;
#pragma unroll
      for (int kk = 0; kk < kBK / 64; kk++) {
        const int co = 16 * ((4 * kk + lq) ^ sw);
        v4i fa[NP][TI], fb[TJ];
#pragma unroll
        for (int p = 0; p < NP; p++)
#pragma unroll
          for (int i = 0; i < TI; i++)
            fa[p][i] = *reinterpret_cast<const v4i *>(ta + (p * BM + 16 * i) * kBK + co);
#pragma unroll
        for (int j = 0; j < TJ; j++) fb[j] = *reinterpret_cast<const v4i *>(tb + bt[j] * kBK + co);
#pragma unroll
        for (int p = 0; p < NP; p++)
#pragma unroll
          for (int i = 0; i < TI; i++)
#pragma unroll
            for (int j = 0; j < TJ; j++) acc[i][j] = Op::mma(fa[p][i], fb[j], acc[i][j]);
      }
    }
  }

  if constexpr (SPLIT) {
    // split K: publish this block's partial tile; the tile's last block adds
    // them.  Device-coherent buffer stores and loads (sc1: they bypass the
    // XCD's L2), a thread's accumulators 16 bytes at a time, and a wait for
    // the stores' completion before the counter, instead of a device-scope
    // fence (which writes back the whole L2).  The last block issues all its
    // loads at once (at most 256 / BM splits, so 128 values per thread):
    // atomic loads came out one round trip each.
    constexpr int NQ = TI * TJ;        // 16-byte accumulator vectors per thread
    constexpr int KSM = 256 / BM;      // splits a launch may use
    const int ks = (int)gridDim.y;
    // the address's halves as unsigned words (readfirstlane returns int: an
    // int low half would sign-extend into the high half)
    const uint64_t pv = (uint64_t)(uintptr_t)(gm_part + (size_t)tl * ks * 256 * NQ * 4);
    const uint32_t plo = __builtin_amdgcn_readfirstlane((uint32_t)pv),
                   phi = __builtin_amdgcn_readfirstlane((uint32_t)(pv >> 32));
    void *pu = (void *)(uintptr_t)(((uint64_t)phi << 32) | plo);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(pu, 0, ks * 256 * NQ * 16, 0x00020000);
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
      for (int j = 0; j < TJ; j++)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, acc[i][j]), rs,
                                               (((int)blockIdx.y * 256 + t) * NQ + i * TJ + j) * 16, 0,
                                               16 /* sc1 */);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __shared__ int s_last;
    __syncthreads();
    if (t == 0)
      s_last = __hip_atomic_fetch_add(&gm_cnt[tl], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ks - 1;
    __syncthreads();
    if (!s_last) return;
    // unconditional loads (splits past ks read the last one again and are
    // not added): behind a branch per split, each split's loads waited for
    // the previous ones
    v4u part[KSM][NQ];
#pragma unroll
    for (int y = 0; y < KSM; y++)
#pragma unroll
      for (int q = 0; q < NQ; q++)
        part[y][q] =
            __builtin_amdgcn_raw_buffer_load_b128(rs, ((min(y, ks - 1) * 256 + t) * NQ + q) * 16, 0, 16 /* sc1 */);
    typedef typename std::conditional<I8, int, float>::type El;
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
      for (int j = 0; j < TJ; j++) {
        El v[4] = {0, 0, 0, 0};
#pragma unroll
        for (int y = 0; y < KSM; y++) {
          // the whole vector cast, then its elements read: a bit cast of an
          // element expression (w.y) read element 0
          const Acc w = __builtin_bit_cast(Acc, part[y][i * TJ + j]);
          if (y < ks) {
            v[0] += w[0];
            v[1] += w[1];
            v[2] += w[2];
            v[3] += w[3];
          }
        }
        // whole-vector assignment: element-wise writes of acc[i][j][r] kept
        // only element 0 of the sums live
        acc[i][j] = Acc{v[0], v[1], v[2], v[3]};
      }
    if (t == 0) __hip_atomic_store(&gm_cnt[tl], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // ---- epilogue: lane holds D[4*lq + r][lr] of each tile ----
  // Every value of a column tile is computed before any of its stores, so
  // that the 4*TI independent chains (SiLU's expf and division, GELU's tanh)
  // interleave instead of each waiting in its own exec-masked branch; tiles
  // wholly inside the matrix store without per-element tests.  Rows and
  // columns past the matrix were loaded clamped: their values are computed
  // and not stored.
  const bool full = m0 + BM <= M && n0 + NOUT <= N;
#pragma unroll
  for (int j = 0; j < JO; j++) {
    const int n = lcol0 + 16 * j;
    const float bs = a.ws ? e_bs[j] : 1.0f;
    const float bv = (!SWI && a.bias) ? e_bv[j] : 0.0f;
    const float bs2 = (SWI && a.ws2) ? e_bs2[j] : 1.0f;
    float v[TI][4];
#pragma unroll
    for (int i = 0; i < TI; i++) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float as = e_as[i][r];
        float x;
        if constexpr (I8) {
          x = i8_epilogue(acc[i][j][r], as, bs, bv);
          if constexpr (SWI) {
            const float u = i8_epilogue(acc[i][j + TJ / 2][r], as, bs2, 0.0f);
            x = silu(x, etab) * u;
          }
        } else {
          // 16-bit: the split's 2^e, then the 16-bit GEMV's epilogue order
          x = acc[i][j][r] * as;
          if constexpr (SWI) {
            const float u = acc[i][j + TJ / 2][r] * as;
            x = silu(x, etab) * u;
          } else if (a.bias) {
            x = x + bv;
          }
        }
        if constexpr (!SWI) {
          if constexpr (RES) x = e_old[i][j][r] + x;
          if constexpr (GELU) x = gelu_new(x);
        }
        v[i][r] = x;
      }
    }
    float *op = a.out + n;
    if (full) {
#pragma unroll
      for (int i = 0; i < TI; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) op[(size_t)(lrow0 + 16 * i + r) * a.ldo] = v[i][r];
    } else if (n < N) {
#pragma unroll
      for (int i = 0; i < TI; i++)
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (lrow0 + 16 * i + r < M) op[(size_t)(lrow0 + 16 * i + r) * a.ldo] = v[i][r];
    }
  }
}

#ifndef EC_GEMM_DL
#define EC_GEMM_DL 1
#endif
// K splits of a launch of T tiles over ns K stages: none when the tiles
// already fill the CUs or the rows are short (under 16 stages: C2's q|k|v,
// o and fc at 12 stages ran 8.6 -> 11.9, 8.6 -> 10.3 and 14.6 -> 18.7 us
// split in 2-3); otherwise up to 256 blocks of 6 stages or more, within the
// partial workspace, and no split left empty.  Only 32-row tiles split (few
// tiles over long rows: a prefill of a few hundred tokens); such a launch
// holds one block per CU and 4 stage buffers.
int gemm_ksplit(int T, int ns, int BM) {
  if (BM != 32 || T >= 128 || ns < 16 || T > kGmMaxTiles) return 1;
  int ks = min(min(ns / 6, 256 / T), 256 / BM);
  ks = min(ks, kGmPartInts / (T * BM * kBN));
  if (ks < 2) return 1;
  const int kper = (ns + ks - 1) / ks;
  return (ns + kper - 1) / kper;
}

template <int OP, int BM, int EPI>
hipError_t launch_bm(const GemvArgs &a, hipStream_t s) {
  constexpr int NOUT = EPI == EPI_SWIGLU ? kBN / 2 : kBN;
  const int T = ((a.N + NOUT - 1) / NOUT) * ((a.M + BM - 1) / BM);
  // split K for few tiles over long rows: C2's 128-token down projection
  // (24 tiles of 32 x 128 over 48 stages of K) ran each tile's whole K on
  // one CU while 232 CUs idled
  const bool dl = EC_GEMM_DL && (a.K * MfmaOp<OP>::EB) % kBK == 0 && (a.lda * MfmaOp<OP>::EB) % kBK == 0;
  const int ks = dl ? gemm_ksplit(T, (a.K * MfmaOp<OP>::EB + kBK - 1) / kBK, BM) : 1;
  const dim3 grid(8 * ((T + 7) / 8), ks);
  if constexpr (BM == 32) {
    static_assert(gemm_lds_bytes<OP, 32, true, 4>() <= 158 * 1024, "split K: 4 stage buffers per CU");
    if (ks > 1) {
      klaunch((gemm_mfma_kernel<OP, 32, EPI, true, 4, true>), grid, dim3(256), gemm_lds_bytes<OP, 32, true, 4>(), s,
              a);
      return hipGetLastError();
    }
  }
  // grids of at most two tiles per CU: the most stage buffers (up to 4) with
  // which the tiles a CU holds at once still fit its LDS, so that 2-3
  // stages' loads are in flight.  C2's 128-token linears (24-96 tiles):
  // down 40.3 -> 23.6 us, q|k|v and o 11.9 -> 8.4 us; C4's down (448
  // tiles) 23.6 -> 21.7 us.
  const int bpc = T * ks <= 256 ? 1 : 2;
  const size_t budget = (size_t)(158 * 1024) / bpc;
  constexpr size_t l4 = gemm_lds_bytes<OP, BM, true, 4>(), l3 = gemm_lds_bytes<OP, BM, true, 3>();
  if (dl && T <= 512 && l4 <= budget)
    klaunch((gemm_mfma_kernel<OP, BM, EPI, true, l4 <= 158 * 1024 ? 4 : 2>), grid, dim3(256),
            gemm_lds_bytes<OP, BM, true, l4 <= 158 * 1024 ? 4 : 2>(), s, a);
  else if (dl && T <= 512 && l3 <= budget)
    klaunch((gemm_mfma_kernel<OP, BM, EPI, true, l3 <= 158 * 1024 ? 3 : 2>), grid, dim3(256),
            gemm_lds_bytes<OP, BM, true, l3 <= 158 * 1024 ? 3 : 2>(), s, a);
  else if (dl) klaunch((gemm_mfma_kernel<OP, BM, EPI, true>), grid, dim3(256), gemm_lds_bytes<OP, BM, true>(), s, a);
  else klaunch((gemm_mfma_kernel<OP, BM, EPI, false>), grid, dim3(256), gemm_lds_bytes<OP, BM, false>(), s, a);
  return hipGetLastError();
}

template <int OP, int EPI>
hipError_t launch_epi(const GemvArgs &a, int bm, hipStream_t s) {
  // the largest row tile that still gives every CU a block or more, else the
  // smallest (N = 896 at M = 2048: 448 blocks of 32 rows beat 224 of 64 rows,
  // 9.7 against 10.7 us for K = 896 and 34.0 against 35.5 us for K = 4864)
  constexpr int NOUT = EPI == EPI_SWIGLU ? kBN / 2 : kBN;
  const long gx = (a.N + NOUT - 1) / NOUT;
  if (bm == 0) bm = gx * ((a.M + 127) / 128) >= 256 ? 128 : gx * ((a.M + 63) / 64) >= 256 ? 64 : 32;
  if (bm == 128) return launch_bm<OP, 128, EPI>(a, s);
  if (bm == 64) return launch_bm<OP, 64, EPI>(a, s);
  return launch_bm<OP, 32, EPI>(a, s);
}

template <int OP>
hipError_t launch_op(const GemvArgs &a, int epi, int bm, hipStream_t s) {
  switch (epi) {
    case EPI_STORE:
    case EPI_BIAS: return launch_epi<OP, EPI_STORE>(a, bm, s);
    case EPI_RESID:
    case EPI_BIAS_RESID: return launch_epi<OP, EPI_RESID>(a, bm, s);
    case EPI_GELU:
    case EPI_BIAS_GELU: return launch_epi<OP, EPI_GELU>(a, bm, s);
    case EPI_SWIGLU: return launch_epi<OP, EPI_SWIGLU>(a, bm, s);
  }
  return hipErrorInvalidValue;
}

bool epi_ok(int epi) {
  return epi == EPI_STORE || epi == EPI_RESID || epi == EPI_GELU || epi == EPI_SWIGLU || epi == EPI_BIAS ||
         epi == EPI_BIAS_RESID || epi == EPI_BIAS_GELU;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// bf16 bits of x rounded to nearest even (finite x)
__device__ __forceinline__ uint16_t f2b_rne(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// one block of 256 threads per row: the row's 16-bit parts and scale
template <int OP>
__global__ __launch_bounds__(256) void split_kernel(const float *x, int ldx, int K, uint16_t *out, int ldo,
                                                    float *rs) {
  __shared__ float red[4];
  const int m = blockIdx.x, t = threadIdx.x;
  const float *row = x + (size_t)m * ldx;
  if constexpr (OP == OP_F16) {
    float mx = 0.0f;
    for (int k = t; k < K; k += 256) mx = fmaxf(mx, fabsf(row[k]));
    mx = block_max256(mx, red);
    // 2^-e x in [2^14, 2^15) for the row's largest |x|; zero, tiny and
    // non-finite rows keep e = 0 (values pass through the fp16 parts)
    int e = 0;
    if (mx > 0.0f && mx <= 3.402823466e38f) e = max(ilogbf(mx) - 14, -100);
    uint16_t *h = out + (size_t)m * 2 * ldo, *l = h + ldo;
    for (int k = t; k < K; k += 256) {
      const float v = ldexpf(row[k], -e);
      const _Float16 hi = (_Float16)v;
      h[k] = __builtin_bit_cast(uint16_t, hi);
      l[k] = f2h(v - (float)hi);
    }
    if (t == 0) rs[m] = ldexpf(1.0f, e);
  } else {
    uint16_t *h = out + (size_t)m * 3 * ldo, *mid = h + ldo, *l = mid + ldo;
    for (int k = t; k < K; k += 256) {
      const float v = row[k];
      const uint16_t b0 = f2b_rne(v);
      const float r1 = v - b2f(b0);
      const uint16_t b1 = f2b_rne(r1);
      const float r2 = r1 - b2f(b1);
      h[k] = b0;
      mid[k] = b1;
      l[k] = f2b_rne(r2);
    }
    if (t == 0) rs[m] = 1.0f;
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// Skinny GEMM (M <= 32 rows: batched decode, a many-row LM head).
//
// One or two 16-row MFMA fragments cover every row, so the weights are the
// whole traffic and the work has to spread over the chip by columns and by K:
// a block owns NJ 16-column output tiles (SwiGLU: the 16 gate and the 16 up
// rows of 16 outputs) and WPB waves (up to 16) that take every WPB-th
// 64-byte K step, each lane loading its MFMA fragments straight from global
// memory (16 bytes of a weight row, 16 bytes of each activation part: the A
// rows stay in L2) with up to 8 steps in flight.  Every block reads all of A
// once, so for wide outputs (the LM head) a block takes 4 tiles and reuses
// each A fragment 4 times.  The waves' partial tiles
// are summed through LDS in wave order (exact for int32) and the block
// applies the epilogue: for int8 the same int32 dots and epilogue code as
// gemm_mfma_kernel, so the same floats; for 16-bit weights the same class of
// fp32 sums.
//
// Split K (int8 only): when the column tiles alone leave most CUs idle
// (down, o and q|k|v at batch 16), gridDim.y blocks share a column group,
// each taking a contiguous range of K steps.  Each writes its int32 tile
// to sk_part, and the last of them to arrive (a counter per column group,
// reset by that block, so every launch finds it at zero) adds the gridDim.y
// tiles and applies the epilogue.  int32 sums are exact in any order, so the
// floats are the same as with one block per column group.  The workspace is
// one per device and the launches that use it must not overlap (the forward
// issues its linears on one stream).
namespace {

constexpr int kSkMaxGroups = 256;              // column groups of a split launch
constexpr int kSkMaxSplit = 8;                 // blocks per column group of a split launch
constexpr int kSkPartInts = 256 * 1024;        // int32 partial tiles of a split launch
__device__ int sk_part[kSkPartInts];
__device__ unsigned sk_cnt[kSkMaxGroups];

// QA (int8 only): A holds fp32 rows, quantized as their fragments are read
// with the row scale quant_scale(max |a|) of the row maximum given as partial
// maxima (a.pmax, a.np); the codes are quant_rows' (the same scale and the
// same per-element code), so the floats equal the unfused GEMM's.
template <int OP, int TI, int NJ, int EPI, bool QA = false>
__global__ __launch_bounds__(1024) void gemm_skinny_kernel(GemvArgs a) {
  using Op = MfmaOp<OP>;
  using Acc = typename Op::Acc;
  constexpr int NP = Op::NP;
  constexpr bool I8 = OP == OP_I8;
  constexpr bool SWI = EPI == EPI_SWIGLU;
  constexpr bool RES = EPI == EPI_RESID || EPI == EPI_BIAS_RESID;
  constexpr bool GELU = EPI == EPI_GELU || EPI == EPI_BIAS_GELU;
  static_assert(!SWI || NJ == 1, "SwiGLU blocks take one tile of gate and up rows");
  static_assert(!QA || I8, "fused quantization of int8 activations");
  constexpr int NB = SWI ? 2 : NJ;  // B tiles: NJ tiles of 16 rows, or 16 gate + 16 up rows
  constexpr int FR = TI * NP * (QA ? 4 : 1) + NB;  // 16-byte loads per lane and step
  constexpr int U = FR <= 3 ? 8 : FR <= 5 ? 4 : 2;  // K steps per wave in flight (within 128 VGPRs)
  __shared__ Acc part[16][TI][NB][64];  // [wave][i][j][lane]
  __shared__ uint64_t etab[SWI ? 32 : 1];
  __shared__ float s_sc[QA ? 32 : 1];  // QA: the rows' scales

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, nw = blockDim.x >> 6;
  const int lr = lane & 15, lq = lane >> 4;
  const int M = a.M, K = a.K, N = a.N;
  const int KB = K * Op::EB;  // bytes of a weight row and of an activation part row
  const size_t ldab = (size_t)a.lda * Op::EB;
  const int n0 = 16 * NJ * blockIdx.x;
  const int ksteps = (KB + 63) / 64;
  if constexpr (SWI) {
    if (t < 32) etab[t] = ec_exp2_32[t];
  }

  // fragment sources: part p of A row 16 i + lr (clamped), B row n0 + lr of W (and W2)
  const int8_t *arow[TI][NP];
  const float *arowf[TI];  // QA: the fp32 row
  const int8_t *brow[NB];
#pragma unroll
  for (int i = 0; i < TI; i++) {
#pragma unroll
    for (int p = 0; p < NP; p++)
      arow[i][p] = (const int8_t *)a.A + ((size_t)min(16 * i + lr, M - 1) * NP + p) * ldab;
    arowf[i] = (const float *)a.A + (size_t)min(16 * i + lr, M - 1) * a.lda;
  }
  // QA: each row's scale from its partial maxima (one wave per row), then
  // this lane's rows' scale and reciprocal
  float qs[TI], qr[TI];
  bool qok[TI];
  if constexpr (QA) {
    // each wave's partial maxima loads of all its rows issued together
    // (kQaLoads per lane and row; np <= 64 kQaLoads)
    constexpr int kQaLoads = 10;
    for (int m0 = wave; m0 < M; m0 += 2 * nw) {
      float pv[2][kQaLoads];
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const int m = min(m0 + nw * h, M - 1);
#pragma unroll
        for (int k = 0; k < kQaLoads; k++) {
          const int j = lane + 64 * k;
          pv[h][k] = j < a.np ? a.pmax[(size_t)m * a.np + j] : 0.0f;
        }
      }
#pragma unroll
      for (int h = 0; h < 2; h++) {
        float mx = 0.0f;
#pragma unroll
        for (int k = 0; k < kQaLoads; k++) mx = fmaxf(mx, pv[h][k]);
        mx = wave_max_dpp(mx);
        if (lane == 0 && m0 + nw * h < M) s_sc[m0 + nw * h] = quant_scale(mx);
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TI; i++) {
      qs[i] = s_sc[min(16 * i + lr, M - 1)];
      qok[i] = ec_quant_rcp_ok(qs[i]);
      qr[i] = qok[i] ? 1.0f / qs[i] : 1.0f;
    }
  }
#pragma unroll
  for (int j = 0; j < NB; j++) {
    if constexpr (SWI) brow[j] = (const int8_t *)(j ? a.W2 : a.W) + (size_t)min(n0 + lr, N - 1) * KB;
    else brow[j] = (const int8_t *)a.W + (size_t)min(n0 + 16 * j + lr, N - 1) * KB;
  }

  Acc acc[TI][NB];
#pragma unroll
  for (int i = 0; i < TI; i++)
#pragma unroll
    for (int j = 0; j < NB; j++) acc[i][j] = Acc{0, 0, 0, 0};

  // this block's K steps [ks0, ks1) (all of them unless K is split)
  const int kper = (ksteps + gridDim.y - 1) / gridDim.y;
  const int ks0 = min(ksteps, kper * (int)blockIdx.y), ks1 = min(ksteps, ks0 + kper);
  // this wave's steps: ks0 + wave, + nw, ... < ks1, U at a time; bytes past
  // the row read a clamped address and the A fragments are zeroed
  for (int sb = ks0 + wave; sb < ks1; sb += nw * U) {
    v4i fa[U][TI][NP], fb[U][NB];
    float4 ff[QA ? U : 1][QA ? TI : 1][4];  // QA: the 16 floats of each A fragment
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int st = sb + nw * u;  // uniform over the wave
      if (st < ks1) {
        const int kc = min(64 * st + 16 * lq, KB - 16);
#pragma unroll
        for (int i = 0; i < TI; i++) {
          if constexpr (QA) {
#pragma unroll
            for (int c = 0; c < 4; c++) ff[u][i][c] = *reinterpret_cast<const float4 *>(arowf[i] + kc + 4 * c);
          } else {
#pragma unroll
            for (int p = 0; p < NP; p++) fa[u][i][p] = *reinterpret_cast<const v4i *>(arow[i][p] + kc);
          }
        }
#pragma unroll
        for (int j = 0; j < NB; j++) fb[u][j] = *reinterpret_cast<const v4i *>(brow[j] + kc);
      }
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int st = sb + nw * u;
      if (st < ks1) {
        const bool in = 64 * st + 16 * lq < KB;
        if constexpr (QA) {
          // the codes of the fragment's 16 elements, packed four per word
#pragma unroll
          for (int i = 0; i < TI; i++) {
            auto pack = [&](auto q1) {
              int w4[4];
#pragma unroll
              for (int c = 0; c < 4; c++) {
                const float e4[4] = {ff[u][i][c].x, ff[u][i][c].y, ff[u][i][c].z, ff[u][i][c].w};
                uint32_t wd = 0;
#pragma unroll
                for (int k = 0; k < 4; k++) wd |= (uint32_t)(uint8_t)q1(e4[k]) << (8 * k);
                w4[c] = (int)wd;
              }
              fa[u][i][0] = v4i{w4[0], w4[1], w4[2], w4[3]};
            };
            // the division-free form for every scale but extreme ones (a
            // branch the lanes of ordinary rows all skip)
            if (qok[i]) pack([&](float e) { return ec_quant1_rcp(e, qs[i], qr[i]); });
            else pack([&](float e) { return quant1(e, qs[i]); });
          }
        }
#pragma unroll
        for (int i = 0; i < TI; i++)
#pragma unroll
          for (int p = 0; p < NP; p++) {
            const v4i av = in ? fa[u][i][p] : v4i{0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < NB; j++) acc[i][j] = Op::mma(av, fb[u][j], acc[i][j]);
          }
      }
    }
  }

  // sum the waves' tiles: thread t < 256 TI NO takes output tile
  // jo = t / (256 TI), fragment i = (t / 256) % TI, accumulator register
  // r = (t / 64) % 4 of lane t % 64, i.e. row 16 i + 4 lq + r, column
  // n0 + 16 jo + lr (SwiGLU: gate and up of that column)
  constexpr int NO = SWI ? 1 : NJ;  // output tiles
#pragma unroll
  for (int i = 0; i < TI; i++)
#pragma unroll
    for (int j = 0; j < NB; j++) part[wave][i][j][lane] = acc[i][j];
  __syncthreads();
  const bool outt = t < 256 * TI * NO;  // an output thread
  const int jo = t / (256 * TI), i = (t >> 8) % TI, r = (t >> 6) & 3;
  const int m = 16 * i + 4 * lq + r, n = n0 + 16 * jo + lr;
  using Sum = std::conditional_t<I8, int, float>;
  constexpr int NS = SWI ? 2 : 1;
  Sum sum[NS];
#pragma unroll
  for (int k = 0; k < NS; k++) {
    const int j = SWI ? k : jo;
    Sum v = 0;
    if (outt) {
      v = part[0][i][j][lane][r];
      for (int w = 1; w < nw; w++) v = v + part[w][i][j][lane][r];
    }
    sum[k] = v;
  }
  if constexpr (I8) {
    if (gridDim.y > 1) {
      // split K: publish this block's tile; the group's last block adds them
      constexpr int TS = 256 * TI * NO * NS;  // ints per tile
      const int ks = (int)gridDim.y;
      // Device-coherent buffer stores and loads (sc1: they bypass the XCD's
      // L2) and a wait for the stores' completion before the counter,
      // instead of fences: a device-scope fence writes back the whole L2
      // (about 50 us per launch measured).  The address's halves as unsigned
      // words (readfirstlane returns int: an int low half would sign-extend
      // into the high half).
      const uint64_t pv = (uint64_t)(uintptr_t)(sk_part + (size_t)blockIdx.x * ks * TS);
      const uint32_t plo = __builtin_amdgcn_readfirstlane((uint32_t)pv),
                     phi = __builtin_amdgcn_readfirstlane((uint32_t)(pv >> 32));
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          (void *)(uintptr_t)(((uint64_t)phi << 32) | plo), 0, ks * TS * 4, 0x00020000);
      if (outt) {
#pragma unroll
        for (int k = 0; k < NS; k++)
          __builtin_amdgcn_raw_buffer_store_b32((uint32_t)sum[k], rs, ((int)blockIdx.y * TS + 256 * TI * NO * k + t) * 4,
                                                0, 16 /* sc1 */);
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __shared__ int s_last;
      __syncthreads();
      if (t == 0)
        s_last = __hip_atomic_fetch_add(&sk_cnt[blockIdx.x], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 gridDim.y - 1;
      __syncthreads();
      if (!s_last) return;
      if (outt) {
        // every split's value loaded at once, unconditionally (splits past
        // ks read the last one again and are not added): atomic loads in a
        // loop came out one round trip each
        uint32_t w[NS][kSkMaxSplit];
#pragma unroll
        for (int k = 0; k < NS; k++)
#pragma unroll
          for (int y = 0; y < kSkMaxSplit; y++)
            w[k][y] = __builtin_amdgcn_raw_buffer_load_b32(rs, (min(y, ks - 1) * TS + 256 * TI * NO * k + t) * 4, 0,
                                                           16 /* sc1 */);
#pragma unroll
        for (int k = 0; k < NS; k++) {
          int v = 0;
#pragma unroll
          for (int y = 0; y < kSkMaxSplit; y++)
            if (y < ks) v += (int)w[k][y];
          sum[k] = v;
        }
      }
      if (t == 0) __hip_atomic_store(&sk_cnt[blockIdx.x], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (!outt) return;
  const bool valid = m < M && n < N;
  if (!valid && !a.pmax_out) return;

  // epilogue (the same code as gemm_mfma_kernel's)
  const float as = QA ? s_sc[min(m, M - 1)] : a.as[min(m, M - 1)];
  float v = 0.0f;
  if (valid) {
  if constexpr (I8) {
    const float bs = a.ws ? a.ws[n] : 1.0f;
    if constexpr (SWI) {
      v = i8_epilogue(sum[0], as, bs, 0.0f);
      const float u = i8_epilogue(sum[1], as, a.ws2 ? a.ws2[n] : 1.0f, 0.0f);
      v = silu(v, etab) * u;
    } else {
      v = i8_epilogue(sum[0], as, bs, a.bias ? a.bias[n] : 0.0f);
    }
  } else {
    v = sum[0] * as;
    if constexpr (SWI) {
      const float u = sum[1] * as;
      v = silu(v, etab) * u;
    } else if (a.bias) {
      v = v + a.bias[n];
    }
  }
  if constexpr (!SWI) {
    if constexpr (RES) v = a.out[(size_t)m * a.ldo + n] + v;
    if constexpr (GELU) v = gelu_new(v);
  }
  a.out[(size_t)m * a.ldo + n] = v;
  }
  if (a.pmax_out) {
    // the largest |v| of row m over this block's 16 NO columns: the 16 lanes
    // of a DPP row hold one row's columns (NaN and absent outputs count 0)
    float pv = valid ? fmaxf(0.0f, fabsf(v)) : 0.0f;
    pv = fmaxf(pv, dpp_mov<0xB1>(pv));
    pv = fmaxf(pv, dpp_mov<0x4E>(pv));
    pv = fmaxf(pv, dpp_mov<0x141>(pv));
    pv = fmaxf(pv, dpp_mov<0x140>(pv));
    if constexpr (NO > 1) {
      __shared__ float s_pm[4][32];  // [tile jo][row]
      if (lr == 0 && m < M) s_pm[jo][m] = pv;
      __syncthreads();
      if (jo == 0 && lr == 0 && m < M) {
        float b = s_pm[0][m];
        for (int q = 1; q < NO; q++) b = fmaxf(b, s_pm[q][m]);
        a.pmax_out[(size_t)m * a.np_out + blockIdx.x] = b;
      }
    } else {
      if (lr == 0 && m < M) a.pmax_out[(size_t)m * a.np_out + blockIdx.x] = pv;
    }
  }
}

template <int OP, int TI, int NJ, int EPI, bool QA = false>
hipError_t launch_skinny_nj(const GemvArgs &a, int wpb, int ksplit, hipStream_t s) {
  const int ksteps = (a.K * MfmaOp<OP>::EB + 63) / 64;
  constexpr int NO = EPI == EPI_SWIGLU ? 1 : NJ;
  const int groups = (a.N + 16 * NJ - 1) / (16 * NJ);
  if (ksplit < 1 || OP != OP_I8 || groups > kSkMaxGroups ||
      (size_t)groups * ksplit * 256 * TI * NO * (EPI == EPI_SWIGLU ? 2 : 1) > (size_t)kSkPartInts)
    ksplit = 1;
  ksplit = min(min(ksplit, ksteps), kSkMaxSplit);
  const int kper = (ksteps + ksplit - 1) / ksplit;
  // waves per block: two or more K steps each (SwiGLU: six), 4 to 16 waves,
  // and at least 4 TI NO (the epilogue takes one thread per output of 16 TI
  // rows x 16 NO).  At batch 16 with weights from HBM (a microbenchmark
  // cycling through more weight copies than the last-level cache holds),
  // gate/up (K = 1536, 24 steps) took 11.0 us with 4 waves against 12.9 us
  // with 12; in the decode 14.1 -> 11.7 us.  The o projection with its fused
  // quantization went the other way (8.5 -> 10.8 us with 4 waves).
  if (wpb <= 0) wpb = min(16, max(4, kper / (EPI == EPI_SWIGLU ? 6 : 2)));
  wpb = max(min(wpb, 16), 4 * TI * NO);
  if (a.pmax_out && groups > a.np_out) return hipErrorInvalidValue;
  klaunch((gemm_skinny_kernel<OP, TI, NJ, EPI, QA>), dim3(groups, ksplit), dim3(64 * wpb), 0, s, a);
  return hipGetLastError();
}

// four column tiles per block for wide outputs (at least 1024 of them), else
// one.  int8 outputs of a long K (64 or more K steps: down at batch 16)
// whose column groups fill less than about 3/4 of the CUs split K over up to
// 8 blocks per group (four column tiles each, so that a block's activation
// fragments serve 64 columns).  The split's publish-and-add round trip costs
// ~3 us, more than it saves for K = 1536 (o and q|k|v at batch 16: 4.7 ->
// 7.2-7.7 us measured); down (K = 8960) goes from 12.6 to 10.2 us.
template <int OP, int TI, int EPI, bool QA = false>
hipError_t launch_skinny(const GemvArgs &a, int wpb, hipStream_t s) {
  if constexpr (EPI != EPI_SWIGLU && TI == 1) {
    if (a.N >= 16 * 1024) return launch_skinny_nj<OP, TI, 4, EPI, QA>(a, wpb, 1, s);
    if (OP == OP_I8 && (a.N + 15) / 16 < 192 && (a.K + 63) / 64 >= 64) {
      const int ksteps = (a.K + 63) / 64, groups = (a.N + 63) / 64;
      const int ks = min(8, min(256 / groups, ksteps / 4));
      if (ks > 1) return launch_skinny_nj<OP, TI, 4, EPI, QA>(a, wpb, ks, s);
    }
  }
  return launch_skinny_nj<OP, TI, 1, EPI, QA>(a, wpb, 1, s);
}

template <int OP, int TI>
hipError_t launch_skinny_epi(const GemvArgs &a, int epi, int wpb, hipStream_t s) {
  switch (epi) {
    case EPI_STORE:
    case EPI_BIAS: return launch_skinny<OP, TI, EPI_STORE>(a, wpb, s);
    case EPI_RESID:
    case EPI_BIAS_RESID: return launch_skinny<OP, TI, EPI_RESID>(a, wpb, s);
    case EPI_GELU:
    case EPI_BIAS_GELU: return launch_skinny<OP, TI, EPI_GELU>(a, wpb, s);
    case EPI_SWIGLU: return launch_skinny<OP, TI, EPI_SWIGLU>(a, wpb, s);
  }
  return hipErrorInvalidValue;
}

template <int OP>
hipError_t launch_skinny_op(const GemvArgs &a, int epi, int wpb, hipStream_t s) {
  return a.M <= 16 ? launch_skinny_epi<OP, 1>(a, epi, wpb, s) : launch_skinny_epi<OP, 2>(a, epi, wpb, s);
}

}  // namespace

bool gemm_i8_ok(const GemvArgs &a, int epi) {
  if (a.M < 1 || a.N < 1 || a.K < 16 || a.K % 16 || a.lda % 16 || !a.as || a.cand) return false;
  if (!aligned16(a.A) || !aligned16(a.W)) return false;
  if (epi == EPI_SWIGLU && (!a.W2 || !aligned16(a.W2))) return false;
  return epi_ok(epi);
}

hipError_t gemm_i8_tile(const GemvArgs &a, int epi, int bm, hipStream_t s) {
  if (!gemm_i8_ok(a, epi) || (bm != 0 && bm != 32 && bm != 64 && bm != 128)) return hipErrorInvalidValue;
  return launch_op<OP_I8>(a, epi, bm, s);
}

hipError_t gemm_i8(const GemvArgs &a, int epi, hipStream_t s) { return gemm_i8_tile(a, epi, 0, s); }

int w16_parts(int wt) { return wt == WT_BF16 ? 3 : 2; }

bool gemm_w16_ok(const GemvArgs &a, int wt, int epi) {
  if (wt != WT_F16 && wt != WT_BF16) return false;
  if (a.M < 1 || a.N < 1 || a.K < 8 || a.K % 8 || a.cand || a.ws || a.ws2) return false;
  if (!aligned16(a.W)) return false;
  if (epi == EPI_SWIGLU && (!a.W2 || !aligned16(a.W2))) return false;
  return epi_ok(epi);
}

hipError_t split_rows16(const GemvArgs &a, int wt, uint16_t *parts, int ldp, float *rs, hipStream_t s) {
  if ((wt != WT_F16 && wt != WT_BF16) || a.M < 1 || a.K < 1) return hipErrorInvalidValue;
  if (!parts || !rs || ldp < a.K || ldp % 8 || !aligned16(parts)) return hipErrorInvalidValue;
  const float *x = (const float *)a.A;
  if (wt == WT_F16) klaunch((split_kernel<OP_F16>), dim3(a.M), dim3(256), 0, s, x, a.lda, a.K, parts, ldp, rs);
  else klaunch((split_kernel<OP_BF16>), dim3(a.M), dim3(256), 0, s, x, a.lda, a.K, parts, ldp, rs);
  return hipGetLastError();
}

hipError_t gemm_w16_parts(const GemvArgs &a, int wt, int epi, int bm, const uint16_t *parts, int ldp,
                          const float *rs, hipStream_t s) {
  if (!gemm_w16_ok(a, wt, epi) || (bm != 0 && bm != 16 && bm != 32 && bm != 64 && bm != 128))
    return hipErrorInvalidValue;
  if (!parts || !rs || ldp < a.K || ldp % 8 || !aligned16(parts)) return hipErrorInvalidValue;
  GemvArgs q = a;
  q.A = parts;
  q.lda = ldp;
  q.as = rs;
  // the 16-bit linears add a bias only in their BIAS epilogues
  if (epi != EPI_BIAS && epi != EPI_BIAS_RESID && epi != EPI_BIAS_GELU) q.bias = nullptr;
  // a wide output (an LM head) at up to 32 rows streams its weights better
  // through the tiled kernel's 32-row tiles: the batch-16 LM head of 151936
  // x 1536 fp16 took 96 us (4.9 TB/s) there against 134 us (3.5 TB/s) in
  // the skinny kernel, whatever its waves per block
  if (bm == 0 && a.M <= 32 && a.N >= 16384) bm = 32;
  if ((bm == 0 && a.M <= 32) || bm == 16) {  // skinny kernel (bm 16 forces it)
    if (a.M > 32) return hipErrorInvalidValue;
    return wt == WT_F16 ? launch_skinny_op<OP_F16>(q, epi, 0, s) : launch_skinny_op<OP_BF16>(q, epi, 0, s);
  }
  return wt == WT_F16 ? launch_op<OP_F16>(q, epi, bm, s) : launch_op<OP_BF16>(q, epi, bm, s);
}

hipError_t gemm_w16_tile(const GemvArgs &a, int wt, int epi, int bm, uint16_t *parts, int ldp, float *rs,
                         hipStream_t s) {
  if (!gemm_w16_ok(a, wt, epi) || (bm != 0 && bm != 16 && bm != 32 && bm != 64 && bm != 128))
    return hipErrorInvalidValue;
  hipError_t e = split_rows16(a, wt, parts, ldp, rs, s);
  if (e != hipSuccess) return e;
  return gemm_w16_parts(a, wt, epi, bm, parts, ldp, rs, s);
}

hipError_t gemm_w16(const GemvArgs &a, int wt, int epi, uint16_t *parts, int ldp, float *rs, hipStream_t s) {
  return gemm_w16_tile(a, wt, epi, 0, parts, ldp, rs, s);
}


hipError_t gemm_i8_skinny(const GemvArgs &a, int epi, int wpb, hipStream_t s) {
  if (!gemm_i8_ok(a, epi) || a.M > 32 || wpb < 0 || wpb > 16) return hipErrorInvalidValue;
  return launch_skinny_op<OP_I8>(a, epi, wpb, s);
}

bool gemm_i8_skinny_q_ok(const GemvArgs &a, int epi) {
  return epi == EPI_RESID && a.M >= 1 && a.M <= 32 && a.N >= 1 && a.K >= 16 && a.K % 16 == 0 && a.lda % 4 == 0 &&
         aligned16(a.A) && aligned16(a.W) && a.pmax && a.np >= 1 && a.np <= 640 && !a.cand;
}

hipError_t gemm_i8_skinny_q(const GemvArgs &a, int epi, hipStream_t s) {
  if (!gemm_i8_skinny_q_ok(a, epi)) return hipErrorInvalidValue;
  return a.M <= 16 ? launch_skinny<OP_I8, 1, EPI_RESID, true>(a, 0, s) : launch_skinny<OP_I8, 2, EPI_RESID, true>(a, 0, s);
}

}  // namespace ec
