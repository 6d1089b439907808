// Causal attention of a prefill: M tokens of one slot at consecutive positions
// p0 .. p0+M-1, whose k / v rows are already in the fp16 cache (RoPE and the
// append ran first).  This is the reference's per-slot prefill loop
// (src/gpt2.c:527-557 GPT-2, 744-777 Qwen2 GQA) with its arithmetic order:
//
//   s_p   = (float)((double)(sequential fp32 sum over d of q_d * k_p[d]) * inv_hd)
//   e_p   = expf(s_p - max_p s_p)           (glibc-exact expf, ec_expf.h)
//   sum   = sum_p (double)e_p
//   pr_p  = (float)((double)e_p * (1 / sum))
//   out_d = sequential fp32 sum over p (ascending) of pr_p * v_p[d]
//
// Every product is rounded before its add, as in the reference's build.  The
// double sum runs in a tree order (lane-strided, then the wave); the
// reference's order differs from it by the last bits of a double, below what
// the float rounding of pr_p resolves except in rare ties.
//
// One block takes one query head and NW * QW consecutive tokens: NW waves of
// QW tokens each (8 x 2 when the scores fit the LDS, else 8 x 1 or 4 x 1).
// The keys of all of them are staged through LDS 64 positions at a time,
// converted to fp32 once for the block:
//   - scores: lane = position; each lane runs its position's sequential dots
//     for the wave's QW tokens off one read of the K row (q in registers); K
//     rows are head_dim + 4 floats apart, so the 16-byte reads of 8 lanes hit
//     distinct banks;
//   - softmax: per token, inside its wave;
//   - output: lane = element d; the wave adds pr_p * v_p[d] for its QW tokens
//     in position order from the staged V rows, the reads of the next four
//     positions issued before the adds of the current four.
// The blocks with the longest key ranges start first; the grid is (head,
// token group), which spreads the blocks over all 8 XCDs.
#include <cfloat>

#include "ec_device.h"
#include "ec_expf.h"
#include "ec_kernels.h"

namespace ec {

namespace {

constexpr int kPfTile = 64;  // positions per staged K / V tile

// NW waves per block, QW tokens per wave (consecutive), NW * QW tokens per block
template <int HD, int NW, int QW>
__global__ __launch_bounds__(NW * 64) void attn_prefill_kernel(AttnArgs a, int ngroups, int nsc) {
  constexpr int NT = NW * 64, QB = NW * QW;
  constexpr int KP = HD + 4;                   // floats per staged row
  constexpr int CPR = HD / 8;                  // 16-byte chunks (8 halves) per cache row
  constexpr int TCH = kPfTile * CPR;           // chunks per tile
  constexpr int NCH = (TCH + NT - 1) / NT;     // chunks per thread
  constexpr int DPL = HD > 64 ? HD / 64 : 1;   // output elements per lane
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float *tile = lds;  // [kPfTile + 4][KP]: K rows, then V rows (4 spare rows for look-ahead reads)
  __shared__ uint64_t etab[32];

  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int h = blockIdx.x;
  const int kvh = h * a.KVH / a.H;
  const int m0 = (ngroups - 1 - (int)blockIdx.y) * QB;  // longest key ranges first
  const int slot = ld_uniform(a.slot + m0);
  const int pos_hi = ld_uniform(a.pos + min(m0 + QB - 1, a.M - 1));
  const int lo0 = a.window > 0 ? max(0, ld_uniform(a.pos + m0) - a.window + 1) : 0;
  // this wave's tokens (tail waves repeat the last token and store nothing)
  int pos[QW], lo[QW], mq[QW];
  bool act[QW];
  float *scq[QW];  // scores, then probabilities, of token i at index p - lo0
#pragma unroll
  for (int i = 0; i < QW; i++) {
    const int m = m0 + QW * w + i;
    act[i] = m < a.M;
    mq[i] = min(m, a.M - 1);
    pos[i] = ld_uniform(a.pos + mq[i]);
    lo[i] = a.window > 0 ? max(0, pos[i] - a.window + 1) : 0;
    scq[i] = lds + (kPfTile + 4) * KP + (QW * w + i) * nsc;
  }
  if (t < 32) etab[t] = ec_exp2_32[t];
  const size_t cbase = (size_t)slot * a.C * a.kv + (size_t)kvh * HD;
  const uint16_t *Kc = a.kc + cbase, *Vc = a.vc + cbase;

  // q rows of the block's tokens through the (still free) tile area into
  // each wave's registers
  for (int e = t; e < QB * HD / 4; e += NT) {
    const int r = e / (HD / 4), c4 = e - r * (HD / 4);
    const float *qrow = a.q + (size_t)min(m0 + r, a.M - 1) * a.ldq + (size_t)h * HD;
    *reinterpret_cast<float4 *>(tile + r * HD + 4 * c4) = *reinterpret_cast<const float4 *>(qrow + 4 * c4);
  }
  __syncthreads();
  float q[QW][HD];
#pragma unroll
  for (int i = 0; i < QW; i++)
#pragma unroll
    for (int c4 = 0; c4 < HD / 4; c4++) {
      const float4 v = *reinterpret_cast<const float4 *>(tile + (QW * w + i) * HD + 4 * c4);
      q[i][4 * c4] = v.x;
      q[i][4 * c4 + 1] = v.y;
      q[i][4 * c4 + 2] = v.z;
      q[i][4 * c4 + 3] = v.w;
    }

  // tile staging: the next tile's 16-byte chunks are loaded into registers
  // (gload) while the waves work on the current one, then converted to fp32
  // into LDS (lstore) after the barrier.  Rows past pos_hi are clamped to it.
  v4u pre[NCH];
  auto gload = [&](const uint16_t *src, int p0) {
#pragma unroll
    for (int j = 0; j < NCH; j++) {
      const int c = min(t + NT * j, TCH - 1), r = c / CPR, cc = c - r * CPR;
      pre[j] = *reinterpret_cast<const v4u *>(src + (size_t)min(p0 + r, pos_hi) * a.kv + 8 * cc);
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int j = 0; j < NCH; j++) {
      const int c = t + NT * j;
      if (TCH % NT == 0 || c < TCH) {
        const int r = c / CPR, cc = c - r * CPR;
        const uint32_t hv[4] = {pre[j].x, pre[j].y, pre[j].z, pre[j].w};
        float f[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          f[2 * i] = h2f((uint16_t)(hv[i] & 0xffffu));
          f[2 * i + 1] = h2f((uint16_t)(hv[i] >> 16));
        }
        float *dst = tile + r * KP + 8 * cc;
        *reinterpret_cast<float4 *>(dst) = make_float4(f[0], f[1], f[2], f[3]);
        *reinterpret_cast<float4 *>(dst + 4) = make_float4(f[4], f[5], f[6], f[7]);
      }
    }
  };

  // ---- scores: lane = position, the QW sequential dots share each K read ----
  float mx[QW];
#pragma unroll
  for (int i = 0; i < QW; i++) mx[i] = -FLT_MAX;
  gload(Kc, lo0);
  for (int p0 = lo0; p0 <= pos_hi; p0 += kPfTile) {
    __syncthreads();  // the previous tile is consumed
    lstore();
    __syncthreads();
    // next K tile, or the first V tile after the last K tile
    if (p0 + kPfTile <= pos_hi) gload(Kc, p0 + kPfTile);
    else gload(Vc, lo0);
    const int p = p0 + lane;
    if (p >= lo[0] && p <= pos[QW - 1]) {
      const float *kr = tile + lane * KP;
      float s[QW];
#pragma unroll
      for (int i = 0; i < QW; i++) s[i] = 0.0f;
#pragma unroll
      for (int c = 0; c < HD / 4; c++) {
        const float4 k4 = *reinterpret_cast<const float4 *>(kr + 4 * c);
        const float kk[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
#pragma unroll
          for (int i = 0; i < QW; i++) {
            const float pr = q[i][4 * c + e] * kk[e];
            s[i] = s[i] + pr;
          }
        }
      }
      // every token's dot is formed in full, interleaved with the others;
      // only the stores below depend on the token's range
#pragma unroll
      for (int i = 0; i < QW; i++) asm volatile("" : "+v"(s[i]));
#pragma unroll
      for (int i = 0; i < QW; i++) {
        if (p >= lo[i] && p <= pos[i]) {
          const float si = (float)((double)s[i] * a.inv_hd);
          scq[i][p - lo0] = si;
          mx[i] = fmaxf(mx[i], si);
        }
      }
    }
  }

  // ---- softmax of each of the wave's tokens ----
  __syncthreads();
#pragma unroll
  for (int i = 0; i < QW; i++) {
    const float m = wave_max_dpp(mx[i]);
    const int n = pos[i] - lo[i] + 1;
    float *sq = scq[i] + (lo[i] - lo0);
    double sum = 0.0;
    for (int k = lane; k < n; k += 64) {
      const float e = ec_expf_tab(sq[k] - m, etab);
      sq[k] = e;
      sum += (double)e;
    }
    sum = wave_sum_dpp(sum);
    const double isum = 1.0 / sum;
    for (int k = lane; k < n; k += 64) sq[k] = (float)((double)sq[k] * isum);
  }

  // ---- output: lane = element d; per token, the sum over positions in order ----
  float o[QW][DPL];
#pragma unroll
  for (int i = 0; i < QW; i++)
#pragma unroll
    for (int j = 0; j < DPL; j++) o[i][j] = 0.0f;
  const int d0 = HD >= 64 ? lane : (lane & (HD - 1));
  for (int p0 = lo0; p0 <= pos_hi; p0 += kPfTile) {
    __syncthreads();  // probabilities written / previous tile consumed
    lstore();
    __syncthreads();
    if (p0 + kPfTile <= pos_hi) gload(Vc, p0 + kPfTile);
    const float *vt = tile + d0;  // staged row of position p at vt + (p - p0) * KP
    // a position that only some tokens of the wave take
    auto add_some = [&](int p) {
      const float *vr = vt + (p - p0) * KP;
#pragma unroll
      for (int i = 0; i < QW; i++) {
        if (p >= lo[i] && p <= pos[i]) {
          const float pr = scq[i][p - lo0];
#pragma unroll
          for (int j = 0; j < DPL; j++) {
            const float pv = pr * vr[64 * j];
            o[i][j] = o[i][j] + pv;
          }
        }
      }
    };
    const int r0 = max(p0, lo[0]), r1 = min(p0 + kPfTile - 1, pos[QW - 1]);
    int c0 = max(p0, lo[QW - 1]), c1 = min(p0 + kPfTile - 1, pos[0]);  // taken by every token
    if (c0 > c1) c0 = r1 + 1, c1 = r1;
    int p = r0;
    for (; p < c0; p++) add_some(p);
    for (; p <= c1 && ((p - lo0) & 3); p++) add_some(p);
    const int ng = p <= c1 ? (c1 - p + 1) >> 2 : 0;
    if (ng > 0) {
      // groups of 4 positions in two register sets (ping-pong): the
      // probabilities (one 16-byte read per token) and V elements of the next
      // group are read before the adds of the current one.  The look-ahead
      // reads are unconditional; past c1 they reach at most 4 positions
      // further: the tile's 4 spare rows, the next token's score slots or the
      // 4 spare floats after the last token's (values not used).
      float4 pa[QW], pb[QW];
      float va[4][DPL], vb[4][DPL];
      auto load4 = [&](int pp, float4 *pr, float (*vv)[DPL]) {
#pragma unroll
        for (int i = 0; i < QW; i++) pr[i] = *reinterpret_cast<const float4 *>(scq[i] + (pp - lo0));
        const float *vr = vt + (pp - p0) * KP;
#pragma unroll
        for (int e = 0; e < 4; e++)
#pragma unroll
          for (int j = 0; j < DPL; j++) vv[e][j] = vr[e * KP + 64 * j];
      };
      auto add4 = [&](const float4 *pr, float (*vv)[DPL]) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
#pragma unroll
          for (int i = 0; i < QW; i++) {
            const float pe = e == 0 ? pr[i].x : e == 1 ? pr[i].y : e == 2 ? pr[i].z : pr[i].w;
#pragma unroll
            for (int j = 0; j < DPL; j++) {
              const float pv = pe * vv[e][j];
              o[i][j] = o[i][j] + pv;
            }
          }
        }
      };
      load4(p, pa, va);
      for (int g = 0;;) {
        load4(p + 4, pb, vb);
        __builtin_amdgcn_sched_barrier(0);
        add4(pa, va);
        __builtin_amdgcn_sched_barrier(0);
        p += 4;
        if (++g == ng) break;
        load4(p + 4, pa, va);
        __builtin_amdgcn_sched_barrier(0);
        add4(pb, vb);
        __builtin_amdgcn_sched_barrier(0);
        p += 4;
        if (++g == ng) break;
      }
    }
    for (; p <= r1; p++) add_some(p);
  }
#pragma unroll
  for (int i = 0; i < QW; i++) {
    if (act[i] && (HD >= 64 || lane < HD)) {
      float *out = a.out + (size_t)mq[i] * a.ldo + (size_t)h * HD + d0;
#pragma unroll
      for (int j = 0; j < DPL; j++) out[64 * j] = o[i][j];
    }
  }
}

// score slots per token: the positions one block reads, window-bounded
int pf_nsc(const AttnArgs &a, int qb) {
  int r = a.max_npos;
  if (a.window > 0 && a.window + qb - 1 < r) r = a.window + qb - 1;
  return (r + 3) & ~3;
}

// tile with 4 spare rows, the score slots of qb tokens and 4 spare floats,
// plus the static expf table (256 bytes)
size_t pf_lds_bytes(const AttnArgs &a, int qb) {
  return ((size_t)(kPfTile + 4) * (a.hd + 4) + (size_t)qb * pf_nsc(a, qb) + 4) * sizeof(float) + 256;
}

// block shapes, largest first: (waves, tokens per wave)
constexpr int kPfShapes[3][2] = {{8, 2}, {8, 1}, {4, 1}};

int pf_pick(const AttnArgs &a, int max_lds) {
  for (int i = 0; i < 3; i++) {
    if (a.hd == 128 && kPfShapes[i][1] > 1) continue;  // two q rows of 128 do not fit the registers
    if (pf_lds_bytes(a, kPfShapes[i][0] * kPfShapes[i][1]) <= (size_t)max_lds) return i;
  }
  return -1;
}

// grid (head, token group): consecutive block ids, which the dispatcher deals
// out to the 8 XCDs in turn, spread every head over every XCD; one slot's K/V
// of all KV heads fits each XCD's L2 at the prefill lengths of the models
template <int HD, int NW, int QW>
void launch_pf(const AttnArgs &a, hipStream_t st) {
  const int ngroups = (a.M + NW * QW - 1) / (NW * QW);
  const dim3 grid(a.H, ngroups);
  klaunch((attn_prefill_kernel<HD, NW, QW>), grid, dim3(NW * 64), pf_lds_bytes(a, NW * QW) - 256, st, a,
          ngroups, pf_nsc(a, NW * QW));
}

template <int HD>
void launch_hd(const AttnArgs &a, int shape, hipStream_t st) {
  if (shape == 0) {
    if constexpr (HD != 128) launch_pf<HD, 8, 2>(a, st);
  } else if (shape == 1) {
    launch_pf<HD, 8, 1>(a, st);
  } else {
    launch_pf<HD, 4, 1>(a, st);
  }
}

}  // namespace

bool attention_prefill_ok(const AttnArgs &a, int max_lds) {
  if (!(a.hd == 32 || a.hd == 64 || a.hd == 128) || !attn_vec(a.hd, a.kv) || a.fuse_kv || a.M < 1) return false;
  if (a.ldq % 4 || ((uintptr_t)a.q & 15u)) return false;  // q rows read as float4
  return pf_pick(a, max_lds) >= 0;
}

hipError_t attention_prefill(const AttnArgs &a, int max_lds, hipStream_t st) {
  if (!attention_prefill_ok(a, max_lds)) return hipErrorInvalidValue;
  const int shape = pf_pick(a, max_lds);
  if (a.hd == 64) launch_hd<64>(a, shape, st);
  else if (a.hd == 128) launch_hd<128>(a, shape, st);
  else launch_hd<32>(a, shape, st);
  return hipGetLastError();
}

}  // namespace ec
