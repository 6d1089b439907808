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
//   - softmax: per token, inside its wave, four of a lane's positions per
//     step (expf without branches);
//   - output: lane = element d; the wave adds pr_p * v_p[d] for its QW tokens
//     in position order from V tiles staged transposed (a lane's positions
//     contiguous, 16-byte reads of four).  A tile that every token of a
//     two-token wave takes whole runs as one asm block whose probabilities
//     come from one read per token and a DPP row broadcast per product;
//     partial tiles read the probabilities by quad, the next quad's reads in
//     flight during the current quad's adds.
// The blocks with the longest key ranges start first; the grid is (head,
// token group), which spreads the blocks over all 8 XCDs.
#include <cfloat>

#include "ec_device.h"
#include "ec_expf.h"
#include "ec_kernels.h"

namespace ec {

namespace {

constexpr int kPfTile = 64;  // positions per staged K / V tile

// The output sums of two tokens over 8*n8 positions (n8 >= 1), in order:
// o_i += pr_i[p] * v[p] (product rounded, then the add) for token i = 0, 1.
// p0/p1: LDS byte addresses of the tokens' probabilities of the first
// position, va: of this lane's element of that position in the transposed V
// tile (all 16-byte aligned).  The reads of the next four positions are in
// flight while the current four are added.  Reads four positions past the end
// (values unused).
__device__ __forceinline__ void pf_chain2(float &o0, float &o1, uint32_t p0, uint32_t p1, uint32_t va, int n8) {
  float t0, t1;
  asm volatile(
      "ds_read_b128 v[40:43], %[p0] offset:0\n"
      "ds_read_b128 v[44:47], %[p1] offset:0\n"
      "ds_read_b128 v[48:51], %[va] offset:0\n"
      "L_pf_chain%=:\n"
      "ds_read_b128 v[52:55], %[p0] offset:16\n"
      "ds_read_b128 v[56:59], %[p1] offset:16\n"
      "ds_read_b128 v[60:63], %[va] offset:16\n"
      "s_waitcnt lgkmcnt(3)\n"
      "v_mul_f32 %[t0], v40, v48\n"
      "v_mul_f32 %[t1], v44, v48\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32 %[t0], v41, v49\n"
      "v_mul_f32 %[t1], v45, v49\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32 %[t0], v42, v50\n"
      "v_mul_f32 %[t1], v46, v50\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32 %[t0], v43, v51\n"
      "v_mul_f32 %[t1], v47, v51\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_add_u32 %[p0], 32, %[p0]\n"
      "v_add_u32 %[p1], 32, %[p1]\n"
      "v_add_u32 %[va], 32, %[va]\n"
      "ds_read_b128 v[40:43], %[p0] offset:0\n"
      "ds_read_b128 v[44:47], %[p1] offset:0\n"
      "ds_read_b128 v[48:51], %[va] offset:0\n"
      "s_waitcnt lgkmcnt(3)\n"
      "v_mul_f32 %[t0], v52, v60\n"
      "v_mul_f32 %[t1], v56, v60\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32 %[t0], v53, v61\n"
      "v_mul_f32 %[t1], v57, v61\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32 %[t0], v54, v62\n"
      "v_mul_f32 %[t1], v58, v62\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32 %[t0], v55, v63\n"
      "v_mul_f32 %[t1], v59, v63\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "s_sub_u32 %[n], %[n], 1\n"
      "s_cmp_lg_u32 %[n], 0\n"
      "s_cbranch_scc1 L_pf_chain%=\n"
      "s_waitcnt lgkmcnt(0)\n"
      : [o0] "+v"(o0), [o1] "+v"(o1), [t0] "=&v"(t0), [t1] "=&v"(t1), [p0] "+v"(p0), [p1] "+v"(p1), [va] "+v"(va),
        [n] "+s"(n8)
      :
      : "v40", "v41", "v42", "v43", "v44", "v45", "v46", "v47", "v48", "v49", "v50", "v51", "v52", "v53", "v54", "v55", "v56", "v57", "v58", "v59", "v60", "v61", "v62", "v63", "scc", "memory");
}

// The output sums of two tokens over one whole tile of 64 positions, in
// order, as pf_chain2.  p0/p1: LDS byte addresses of the tokens'
// probabilities of positions 4*(lane % 16) .. +3 of the tile, so that lane j
// of every 16-lane row holds those of quad j; each product takes its
// probability from that lane by a DPP row broadcast (row_newbcast), which
// replaces a 64-lane broadcast read per quad and token.  va: LDS byte address
// of this lane's element of the tile's first position in the transposed V
// tile; quad j is read 16*j bytes further, eight quads ahead of its adds.
__device__ __forceinline__ void pf_tile2(float &o0, float &o1, uint32_t p0, uint32_t p1, uint32_t va) {
  float t0, t1;
  asm volatile(
      "ds_read_b128 v[40:43], %[p0]\n"
      "ds_read_b128 v[44:47], %[p1]\n"
      "ds_read_b128 v[48:51], %[va] offset:0\n"
      "ds_read_b128 v[52:55], %[va] offset:16\n"
      "ds_read_b128 v[56:59], %[va] offset:32\n"
      "ds_read_b128 v[60:63], %[va] offset:48\n"
      "ds_read_b128 v[64:67], %[va] offset:64\n"
      "ds_read_b128 v[68:71], %[va] offset:80\n"
      "ds_read_b128 v[72:75], %[va] offset:96\n"
      "ds_read_b128 v[76:79], %[va] offset:112\n"
      "s_waitcnt lgkmcnt(7)\n"
      "v_mul_f32_dpp %[t0], v40, v48 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v44, v48 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v41, v49 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v45, v49 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v42, v50 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v46, v50 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v43, v51 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v47, v51 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "ds_read_b128 v[48:51], %[va] offset:128\n"
      "s_waitcnt lgkmcnt(7)\n"
      "v_mul_f32_dpp %[t0], v40, v52 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v44, v52 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v41, v53 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v45, v53 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v42, v54 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v46, v54 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v43, v55 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v47, v55 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "ds_read_b128 v[52:55], %[va] offset:144\n"
      "s_waitcnt lgkmcnt(7)\n"
      "v_mul_f32_dpp %[t0], v40, v56 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v44, v56 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v41, v57 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v45, v57 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v42, v58 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v46, v58 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v43, v59 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v47, v59 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "ds_read_b128 v[56:59], %[va] offset:160\n"
      "s_waitcnt lgkmcnt(7)\n"
      "v_mul_f32_dpp %[t0], v40, v60 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v44, v60 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v41, v61 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v45, v61 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v42, v62 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v46, v62 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v43, v63 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v47, v63 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "ds_read_b128 v[60:63], %[va] offset:176\n"
      "s_waitcnt lgkmcnt(7)\n"
      "v_mul_f32_dpp %[t0], v40, v64 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v44, v64 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v41, v65 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v45, v65 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v42, v66 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v46, v66 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v43, v67 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v47, v67 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "ds_read_b128 v[64:67], %[va] offset:192\n"
      "s_waitcnt lgkmcnt(7)\n"
      "v_mul_f32_dpp %[t0], v40, v68 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v44, v68 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v41, v69 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v45, v69 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v42, v70 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v46, v70 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v43, v71 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v47, v71 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "ds_read_b128 v[68:71], %[va] offset:208\n"
      "s_waitcnt lgkmcnt(7)\n"
      "v_mul_f32_dpp %[t0], v40, v72 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v44, v72 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v41, v73 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v45, v73 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v42, v74 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v46, v74 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v43, v75 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v47, v75 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "ds_read_b128 v[72:75], %[va] offset:224\n"
      "s_waitcnt lgkmcnt(7)\n"
      "v_mul_f32_dpp %[t0], v40, v76 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v44, v76 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v41, v77 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v45, v77 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v42, v78 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v46, v78 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v43, v79 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v47, v79 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "ds_read_b128 v[76:79], %[va] offset:240\n"
      "s_waitcnt lgkmcnt(7)\n"
      "v_mul_f32_dpp %[t0], v40, v48 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v44, v48 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v41, v49 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v45, v49 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v42, v50 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v46, v50 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v43, v51 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v47, v51 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "s_waitcnt lgkmcnt(6)\n"
      "v_mul_f32_dpp %[t0], v40, v52 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v44, v52 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v41, v53 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v45, v53 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v42, v54 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v46, v54 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v43, v55 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v47, v55 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "s_waitcnt lgkmcnt(5)\n"
      "v_mul_f32_dpp %[t0], v40, v56 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v44, v56 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v41, v57 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v45, v57 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v42, v58 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v46, v58 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v43, v59 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v47, v59 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_mul_f32_dpp %[t0], v40, v60 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v44, v60 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v41, v61 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v45, v61 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v42, v62 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v46, v62 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v43, v63 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v47, v63 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "s_waitcnt lgkmcnt(3)\n"
      "v_mul_f32_dpp %[t0], v40, v64 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v44, v64 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v41, v65 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v45, v65 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v42, v66 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v46, v66 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v43, v67 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v47, v67 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "s_waitcnt lgkmcnt(2)\n"
      "v_mul_f32_dpp %[t0], v40, v68 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v44, v68 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v41, v69 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v45, v69 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v42, v70 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v46, v70 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v43, v71 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v47, v71 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "s_waitcnt lgkmcnt(1)\n"
      "v_mul_f32_dpp %[t0], v40, v72 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v44, v72 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v41, v73 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v45, v73 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v42, v74 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v46, v74 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v43, v75 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v47, v75 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "s_waitcnt lgkmcnt(0)\n"
      "v_mul_f32_dpp %[t0], v40, v76 row_newbcast:15 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v44, v76 row_newbcast:15 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v41, v77 row_newbcast:15 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v45, v77 row_newbcast:15 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v42, v78 row_newbcast:15 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v46, v78 row_newbcast:15 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      "v_mul_f32_dpp %[t0], v43, v79 row_newbcast:15 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %[t1], v47, v79 row_newbcast:15 row_mask:0xf bank_mask:0xf\n"
      "v_add_f32 %[o0], %[o0], %[t0]\n"
      "v_add_f32 %[o1], %[o1], %[t1]\n"
      : [o0] "+v"(o0), [o1] "+v"(o1), [t0] "=&v"(t0), [t1] "=&v"(t1)
      : [p0] "v"(p0), [p1] "v"(p1), [va] "v"(va)
      : "v40", "v41", "v42", "v43", "v44", "v45", "v46", "v47", "v48", "v49", "v50", "v51", "v52", "v53", "v54", "v55", "v56", "v57", "v58", "v59", "v60", "v61", "v62", "v63", "v64", "v65", "v66", "v67", "v68", "v69", "v70", "v71", "v72", "v73", "v74", "v75", "v76", "v77", "v78", "v79", "memory");
}

// V tiles are staged transposed: element d of the tile's position r at
// tile[pf_vrow(d) + r].  Rows are 68 floats apart plus 4 more every 8 rows,
// so that the 4-byte staging writes (32 lanes: 4 positions x 8 chunks of 8
// elements) and the 16-byte reads of 8 consecutive rows (served 8 lanes at a
// time) both hit distinct banks.
constexpr int pf_vrow(int d) { return d * (kPfTile + 4) + 4 * (d >> 3); }

// NW waves per block, QW tokens per wave (consecutive), NW * QW tokens per block
template <int HD, int NW, int QW>
__global__ __launch_bounds__(NW * 64) void attn_prefill_kernel(AttnArgs a, int ngroups, int nsc) {
  constexpr int NT = NW * 64, QB = NW * QW;
  constexpr int KP = HD + 4;                   // floats per staged row
  constexpr int CPR = HD / 8;                  // 16-byte chunks (8 halves) per cache row
  constexpr int TCH = kPfTile * CPR;           // chunks per tile
  constexpr int NCH = (TCH + NT - 1) / NT;     // chunks per thread
  constexpr int DPL = HD > 64 ? HD / 64 : 1;   // output elements per lane
  constexpr int VJ = pf_vrow(64);              // transposed V: element d + 64 is VJ floats after d
  static_assert(pf_vrow(HD - 1) + kPfTile + 4 <= (kPfTile + 4) * KP, "transposed V tile fits the tile area");
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float *tile = lds;  // [kPfTile + 4][KP]: K rows (4 spare rows for look-ahead reads), then transposed V
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
  // into LDS after the barrier, K row by row (lstore), V transposed
  // (lstore_v).  Rows past pos_hi are clamped to it.
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
        // the row's two halves in the opposite order for chunks 4-7: the 8
        // lanes of one row then write 8 distinct slots mod 8 per instruction
        // (16-byte accesses are served 8 lanes at a time)
        float *dst = tile + r * KP + 8 * cc;
        const bool sw = cc & 4;
        *reinterpret_cast<float4 *>(dst + (sw ? 4 : 0)) =
            sw ? make_float4(f[4], f[5], f[6], f[7]) : make_float4(f[0], f[1], f[2], f[3]);
        *reinterpret_cast<float4 *>(dst + (sw ? 0 : 4)) =
            sw ? make_float4(f[0], f[1], f[2], f[3]) : make_float4(f[4], f[5], f[6], f[7]);
      }
    }
  };
  auto lstore_v = [&]() {
#pragma unroll
    for (int j = 0; j < NCH; j++) {
      const int c = t + NT * j;
      if (TCH % NT == 0 || c < TCH) {
        const int r = c / CPR, cc = c - r * CPR;
        const uint32_t hv[4] = {pre[j].x, pre[j].y, pre[j].z, pre[j].w};
        // elements 8cc .. 8cc+7 share d >> 3: rows kPfTile + 4 floats apart
        float *dst = tile + pf_vrow(8 * cc) + r;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          dst[(2 * i) * (kPfTile + 4)] = h2f((uint16_t)(hv[i] & 0xffffu));
          dst[(2 * i + 1) * (kPfTile + 4)] = h2f((uint16_t)(hv[i] >> 16));
        }
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
    // four of the lane's scores per step, k, k + 64, k + 128, k + 192 (the
    // lane's order of its part of the sum); past n a score of -inf adds
    // exp = 0 (reads clamped to the token's last slot)
    double sum = 0.0;
    for (int k = lane; k < n; k += 256) {
      float e[4];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const float v = sq[min(k + 64 * u, n - 1)];
        e[u] = k + 64 * u < n ? v - m : -__builtin_inff();
      }
#pragma unroll
      for (int u = 0; u < 4; u++) e[u] = ec_expf_tab(e[u], etab);
#pragma unroll
      for (int u = 0; u < 4; u++) {
        if (k + 64 * u < n) sq[k + 64 * u] = e[u];
        sum += (double)e[u];
      }
    }
    sum = wave_sum_dpp(sum);
    const double isum = 1.0 / sum;
    for (int k = lane; k < n; k += 256) {
      float v[4];
#pragma unroll
      for (int u = 0; u < 4; u++) v[u] = sq[min(k + 64 * u, n - 1)];
#pragma unroll
      for (int u = 0; u < 4; u++)
        if (k + 64 * u < n) sq[k + 64 * u] = (float)((double)v[u] * isum);
    }
  }

  // ---- output: lane = element d; per token, the sum over positions in order ----
  float o[QW][DPL];
#pragma unroll
  for (int i = 0; i < QW; i++)
#pragma unroll
    for (int j = 0; j < DPL; j++) o[i][j] = 0.0f;
  const int d0 = HD >= 64 ? lane : (lane & (HD - 1));
  // this lane's element of the tile's position p at vt[p - p0] (of element
  // d0 + 64 j at vt[p - p0 + VJ * j])
  const float *vt = tile + pf_vrow(d0);
  for (int p0 = lo0; p0 <= pos_hi; p0 += kPfTile) {
    __syncthreads();  // probabilities written / previous tile consumed
    lstore_v();
    __syncthreads();
    if (p0 + kPfTile <= pos_hi) gload(Vc, p0 + kPfTile);
    // a position that only some tokens of the wave take
    auto add_some = [&](int p) {
      const float *vr = vt + (p - p0);
#pragma unroll
      for (int i = 0; i < QW; i++) {
        if (p >= lo[i] && p <= pos[i]) {
          const float pr = scq[i][p - lo0];
#pragma unroll
          for (int j = 0; j < DPL; j++) {
            const float pv = pr * vr[VJ * j];
            o[i][j] = o[i][j] + pv;
          }
        }
      }
    };
    const int r0 = max(p0, lo[0]), r1 = min(p0 + kPfTile - 1, pos[QW - 1]);
    int c0 = max(p0, lo[QW - 1]), c1 = min(p0 + kPfTile - 1, pos[0]);  // taken by every token
    if constexpr (QW == 2 && DPL == 1) {
      if (c0 == p0 && c1 == p0 + kPfTile - 1) {  // the whole tile, for both tokens
        const int pq = p0 - lo0 + 4 * (lane & 15);
        pf_tile2(o[0][0], o[1][0], (uint32_t)(uintptr_t)(scq[0] + pq), (uint32_t)(uintptr_t)(scq[QW - 1] + pq),
                 (uint32_t)(uintptr_t)vt);
        continue;
      }
    }
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
      if constexpr (QW == 2 && DPL == 1) {
        // the two-token, one-element case (the long prompts) in one asm loop
        // of 8 positions per iteration; an odd group and the tail below
        const int n8 = __builtin_amdgcn_readfirstlane(ng >> 1);
        if (n8 > 0) {
          pf_chain2(o[0][0], o[1][0], (uint32_t)(uintptr_t)(scq[0] + (p - lo0)),
                    (uint32_t)(uintptr_t)(scq[QW - 1] + (p - lo0)), (uint32_t)(uintptr_t)(vt + (p - p0)), n8);
          p += 8 * n8;
        }
        for (int e = 0; e < 4 * (ng & 1); e++, p++) add_some(p);
      } else {
      float4 pa[QW], pb[QW];
      float va[4][DPL], vb[4][DPL];
      auto load4 = [&](int pp, float4 *pr, float (*vv)[DPL]) {
#pragma unroll
        for (int i = 0; i < QW; i++) pr[i] = *reinterpret_cast<const float4 *>(scq[i] + (pp - lo0));
        const float *vr = vt + (pp - p0);
#pragma unroll
        for (int j = 0; j < DPL; j++) {
          const float4 v4 = *reinterpret_cast<const float4 *>(vr + VJ * j);
          vv[0][j] = v4.x;
          vv[1][j] = v4.y;
          vv[2][j] = v4.z;
          vv[3][j] = v4.w;
        }
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
