// Causal GQA prefill for long prompts on fp16 MFMA, two query heads per wave: every K and V operand read from LDS
// feeds two MFMAs.
//
// Semantics follow attn_split.comp:9-58 + attn_combine.comp:6-21 + gate_rotate.comp:19-25 of the reference, as
// prefill_kernel (same arguments, same results within fp32 rounding): row t (position off+t) of head h attends to
// cache rows [0, off+t+1) of kv head h/4; softmax(q.k/16) v, then a * sigmoid(gate), optionally rotated. q comes as
// fp16 bits.
//
// Decomposition (this kernel's own):
//   One block per q-tile (32 tokens x the 4 query heads of one kv head), 4 waves, one per SIMD, each with the SIMD's
//   whole register file. Wave w holds the head pair 2 (w % 2), 2 (w % 2) + 1 over the q-tile's 32 tokens: 64 query
//   rows, O in all 256 accumulation registers (2 heads x 8 tiles of 32 x 32 fp32), Q^T in 128 VGPRs. Waves 0-1 (group
//   0) attend to the first half of the q-tile's key tiles, waves 2-3 (group 1) to the second half; the two partial
//   (m, l, O) merge through LDS at the end. With whole q-tiles per block a 4,096-token prompt would leave the short
//   q-tiles' CUs idle; with the halves a block costs half its key range, and blocks issued longest first pair up (long
//   + short) on each CU over the launch's two rounds.
//   Per 32-key tile a wave issues 32 MFMAs for S^T = K Q^T (one K operand read per two MFMAs) and 32 for O += P V (one
//   transposed V read per two MFMAs): half the LDS bytes per MFMA of one head per wave, which is what lets one wave
//   per SIMD keep the matrix cores fed (a wave's LDS reads alone cannot feed one head per wave at full rate).
//   Pipeline per tile j: S^T(j) on the MFMA units, then O += P(j - 1) V(j - 1) on the MFMA units while the VALU turns
//   S^T(j) into P(j). K and V have separate 2-stage rings per group in LDS (prefill_kernel's padded row-pair layout);
//   K(j + 1) is copied during the S^T phase of tile j and V(j) during its PV phase (global_load_lds, no VGPRs), each
//   waited for one phase before it is read.
//   The loop is assembly with a fixed register map (bn_prefill_pair_loop.h): a wave's O, Q^T, S^T and P take about 490
//   of its 512 registers, more than the compiler's allocator placed without spilling.
//   Softmax in fp32, log2 domain; the running max moves only when a row's max grows by more than 2^8, so O is rarely
//   rescaled. The row sums add the fp16-rounded probabilities (v_dot2_f32_f16), the values the PV product uses.
//   Causal masking only on tiles that cross the diagonal; tiles past it are not visited.
#pragma once
#include "bn_prefill.h"
#include "bn_prefill_pair_loop.h"

namespace bn {

constexpr int PP_GROUP = 2 * PF_KB + 2 * PF_VB;  // one wave group's LDS: two K stages, two V stages (68,096 B)
constexpr int PP_XSLOT = 32768;                  // O handed over per wave at the merge: 2 heads x 4 tiles x 32 x 32 fp32
constexpr int PP_OP = 1040;                      // row pitch (bytes) of the merged output rows in LDS

// clobber lists of the loop: v0-v223, v240-v255, s80-s97
#define PP_V10(x) "v" #x "0", "v" #x "1", "v" #x "2", "v" #x "3", "v" #x "4", "v" #x "5", "v" #x "6", "v" #x "7", "v" #x "8", "v" #x "9"
#define PP_CLOBBERS                                                                                                    \
    "v0", "v1", "v2", "v3", "v4", "v5", "v6", "v7", "v8", "v9", PP_V10(1), PP_V10(2), PP_V10(3), PP_V10(4), PP_V10(5),  \
        PP_V10(6), PP_V10(7), PP_V10(8), PP_V10(9), PP_V10(10), PP_V10(11), PP_V10(12), PP_V10(13), PP_V10(14),        \
        PP_V10(15), PP_V10(16), PP_V10(17), PP_V10(18), PP_V10(19), PP_V10(20), PP_V10(21), "v220", "v221", "v222",     \
        "v223", PP_V10(24), "v250", "v251", "v252", "v253", "v254", "v255", "s80", "s81", "s82", "s83", "s84", "s85",   \
        "s86", "s87", "s88", "s89", "s90", "s91", "s92", "s93", "s94", "s95", "s96", "s97", "s79", "s70", "s71", "s72", "s73", "vcc", "memory"

// O = 0 in the accumulation registers the loop uses (tile (head hh, dims 32 dt ..) in a[16 (8 hh + dt) : +15])
__device__ __forceinline__ void pp_zero_o(f16x (&o)[2][8]) {
    asm volatile(R"ASM(
  .set ppz_a, 0
  .rept 256
    v_accvgpr_write_b32 a[ppz_a], 0
    .set ppz_a, ppz_a + 1
  .endr
)ASM"
                 : "={a[0:15]}"(o[0][0]), "={a[16:31]}"(o[0][1]), "={a[32:47]}"(o[0][2]), "={a[48:63]}"(o[0][3]),
                   "={a[64:79]}"(o[0][4]), "={a[80:95]}"(o[0][5]), "={a[96:111]}"(o[0][6]), "={a[112:127]}"(o[0][7]),
                   "={a[128:143]}"(o[1][0]), "={a[144:159]}"(o[1][1]), "={a[160:175]}"(o[1][2]),
                   "={a[176:191]}"(o[1][3]), "={a[192:207]}"(o[1][4]), "={a[208:223]}"(o[1][5]),
                   "={a[224:239]}"(o[1][6]), "={a[240:255]}"(o[1][7]));
}

#define PP_O_INPUTS(o)                                                                                                 \
    "{a[0:15]}"(o[0][0]), "{a[16:31]}"(o[0][1]), "{a[32:47]}"(o[0][2]), "{a[48:63]}"(o[0][3]), "{a[64:79]}"(o[0][4]),   \
        "{a[80:95]}"(o[0][5]), "{a[96:111]}"(o[0][6]), "{a[112:127]}"(o[0][7]), "{a[128:143]}"(o[1][0]),                \
        "{a[144:159]}"(o[1][1]), "{a[160:175]}"(o[1][2]), "{a[176:191]}"(o[1][3]), "{a[192:207]}"(o[1][4]),             \
        "{a[208:223]}"(o[1][5]), "{a[224:239]}"(o[1][6]), "{a[240:255]}"(o[1][7])

// One head's O (head HH of the wave's pair) into the merged-row staging, straight from the accumulation registers:
// register r of tile (HH, dims 32 dt ..) at obase + (32 HH + 8 (r / 4) + r % 4) PP_OP + 128 dt. The loop's last
// products have written O first (32 wait states).
template <int HH>
__device__ __forceinline__ void pp_dump_o(f16x (&o)[2][8], uint32_t obase) {
    asm volatile(R"ASM(
  s_nop 7
  s_nop 7
  s_nop 7
  s_nop 7
  .irp dt, 0,1,2,3,4,5,6,7
    .irp r, 0,1,2,3,4,5,6,7,8,9,10,11,12,13,14,15
      ds_write_b32 %[ob], a[16*(8*%[hh]+\dt)+\r] offset:(32*%[hh]+8*((\r)>>2)+((\r)&3))*1040+128*\dt
    .endr
  .endr
  s_waitcnt lgkmcnt(0)
)ASM" ::[ob] "v"(obase), [hh] "n"(HH), PP_O_INPUTS(o)
                 : "memory");
}
// The merge of head HH in place: staging = O fo + staging fx per row (O: this wave's, staging: the partner's dump),
// the 16 factors of a lane's register rows read from bc (fo at bc + 32 q + 16 (l / 32) into v32-v47, fx 128 bytes on
// into v48-v63). The partner's values of dim tile dt + 1 are requested (into the other half of v0-v31) as soon as
// tile dt's have landed, so their latency passes under tile dt's arithmetic; every wait drains the LDS counter.
template <int HH>
__device__ __forceinline__ void pp_merge_o(f16x (&o)[2][8], uint32_t obase, uint32_t bc) {
    asm volatile(R"ASM(
  s_nop 7
  s_nop 7
  s_nop 7
  s_nop 7
  .irp q, 0,1,2,3
    ds_read_b128 v[32+4*\q:35+4*\q], %[bc] offset:32*\q
    ds_read_b128 v[48+4*\q:51+4*\q], %[bc] offset:128+32*\q
  .endr
  .irp r, 0,1,2,3,4,5,6,7,8,9,10,11,12,13,14,15
    ds_read_b32 v[\r], %[ob] offset:(32*%[hh]+8*((\r)>>2)+((\r)&3))*1040
  .endr
  .irp dt, 0,1,2,3,4,5,6,7
    s_waitcnt lgkmcnt(0)
    .if \dt < 7
      .irp r, 0,1,2,3,4,5,6,7,8,9,10,11,12,13,14,15
        ds_read_b32 v[16*(((\dt)+1)&1)+\r], %[ob] offset:(32*%[hh]+8*((\r)>>2)+((\r)&3))*1040+128*(\dt+1)
      .endr
    .endif
    .irp r, 0,1,2,3,4,5,6,7,8,9,10,11,12,13,14,15
      v_accvgpr_read_b32 v[64+((\r)&7)], a[16*(8*%[hh]+\dt)+\r]
      v_mul_f32 v[64+((\r)&7)], v[64+((\r)&7)], v[32+\r]
      v_fmac_f32 v[64+((\r)&7)], v[16*((\dt)&1)+\r], v[48+\r]
      ds_write_b32 %[ob], v[64+((\r)&7)] offset:(32*%[hh]+8*((\r)>>2)+((\r)&3))*1040+128*\dt
    .endr
  .endr
  s_waitcnt lgkmcnt(0)
)ASM" ::[ob] "v"(obase), [bc] "v"(bc), [hh] "n"(HH), PP_O_INPUTS(o)
                 : "v0", "v1", "v2", "v3", "v4", "v5", "v6", "v7", "v8", "v9", PP_V10(1), PP_V10(2), PP_V10(3),
                   PP_V10(4), PP_V10(5), PP_V10(6), "v70", "v71", "memory");
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void prefill_pair_kernel(PrefillArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * PP_GROUP];
    __shared__ float ml_lds[4][2][2][32];  // per wave, head of its pair: m, l of the head's 32 rows
    __shared__ f4 bc_lds[4][2][2][8];      // per wave, head, factor: 32 floats broadcast in row order
    __shared__ float al_lds[4][2][32];     // per wave, head: the loop's rescale factors by row

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), g = w >> 1, pr = w & 1;  // wave-uniform
    const int h = lane >> 5, r32 = lane & 31;
    const int KV = a.KV, ntq = a.ntq;

    // block -> (kv head, q-tile): longest q-tiles (highest index) first, each kv head on a fixed set of XCDs
    int kh, qt;
    {
        const int b = blockIdx.x, nb = KV * ntq;
        int idx;
        if (8 % KV == 0 && nb % 8 == 0) {
            const int xcd = b & 7, reps = 8 / KV;
            kh = xcd % KV;
            idx = (b >> 3) * reps + xcd / KV;
        } else {
            kh = b % KV;
            idx = b / KV;
        }
        qt = ntq - 1 - idx;
    }
    const int t0 = qt * PF_BQ;
    const int t_last = min(a.T, t0 + PF_BQ) - 1;
    const int off = call_off(a.dyn, a.off);
    const int nk = off + a.T;                          // cache rows that exist
    const int nt = (off + t_last + PF_BK) / PF_BK;     // key tiles the q-tile attends to
    const int half = (nt + 1) >> 1;
    const int jb = g ? half : 0;                       // this group's first key tile ...
    const int n = g ? nt - half : half;                // ... and its tile count (group 1 may have one fewer, or none)
    const int64_t kvd = (int64_t)KV * D;
    const uint16_t* kb = a.kc + (int64_t)kh * D;
    const uint16_t* vb = a.vc + (int64_t)kh * D;

    // the group's rings (LDS byte addresses): K stages kst0, kst1, V stages vst0, vst1; a wave copies row pairs
    // 8 pr .. 8 pr + 7 of each tile
    auto la = [](const void* p) { return (uint32_t)(uintptr_t)(pf_lds_void_t*)p; };
    uint8_t* const gl = lds + g * PP_GROUP;
    const uint32_t kr0 = la(gl), kr1 = kr0 + PF_KB, vr0 = kr0 + 2 * PF_KB, vr1 = vr0 + PF_VB;
    const uint32_t kc0 = kr0 + 8 * pr * PF_KP, kc1 = kr1 + 8 * pr * PF_KP;
    const uint32_t vc0 = vr0 + 8 * pr * PF_VP, vc1 = vr1 + 8 * pr * PF_VP;
    const uint64_t kbp = (uint64_t)(uintptr_t)kb, vbp = (uint64_t)(uintptr_t)vb;
    const uint32_t klo = (uint32_t)kbp, khi = (uint32_t)(kbp >> 32), vlo = (uint32_t)vbp, vhi = (uint32_t)(vbp >> 32);
    const uint32_t rowb = (uint32_t)(kvd * 2), pr8 = 8 * pr, offt0 = off + t0;
    const uint32_t un = n, uhalf = half, ujb = jb, unk = nk;

    // per-lane inputs of the loop
    const uint32_t k_lane = (r32 & 15) * PF_KP + (r32 >> 4) * 512 + h * 16;
    const int vs = lane & 15, vnh = (lane >> 4) & 1;
    const uint32_t v_lane = (4 * h + (vs >> 2)) * PF_VP + 32 * vnh + 8 * (vs & 3);
    const uint32_t lane_go = (uint32_t)(16 * h * (int)kvd + r32 * 8) * 2u;
    const int limbase = off + t0 + r32 - 4 * h;        // register r holds key j0 + 8 (r / 4) + 4 h + r % 4 <= qpos
    const uint32_t bcw = la(&al_lds[w][0][0]) + 4 * r32, bcr = la(&al_lds[w][0][0]) + 16 * h;
    const uint32_t h16 = 16 * h, r16 = 16 * r32;

    f16x o[2][8];
    pp_zero_o(o);
    // the group's first key tile into K stage 0 (row pairs 8 pr .. 8 pr + 7; rows past the cache clamp to its last)
    if (n > 0) {
        const int j0 = jb * PF_BK, lim = nk - 1 - j0;
        const char* kt = reinterpret_cast<const char*>(kb + (int64_t)j0 * kvd);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int p = 8 * pr + i;
            const uint32_t go = (uint32_t)(min(p + 16 * h, lim) * (int)kvd + r32 * 8) * 2u;
            __builtin_amdgcn_global_load_lds(kt + go, (pf_lds_void_t*)(gl + p * PF_KP), 16, 0, 0);
        }
    }
    // Q rows of the block (4 heads x 32 tokens, fp16), two whole rows per load, staged behind each group's K stage 0
    // (heads 2p, 2p + 1 in group p's area, pitch PF_QP); the loop's first copies overwrite them after its first barrier
    {
        u4 x[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int tl = min(t0 + 2 * i + h, a.T - 1);  // block row 32 w + 2 i + h: head w, token 2 i + h
            x[i] = *reinterpret_cast<const u4*>(a.q16 + (int64_t)tl * a.q_ts + (int64_t)(kh * 4 + w) * a.q_hs + 8 * r32);
        }
        uint8_t* const qs = lds + (w >> 1) * PP_GROUP + PF_KB + ((w & 1) * 32 + h) * PF_QP + 16 * r32;
#pragma unroll
        for (int i = 0; i < 16; i++) *reinterpret_cast<u4*>(qs + 2 * i * PF_QP) = x[i];
    }
    __syncthreads();
    // Q^T operand of head 2 pr + hh: lane l holds token l % 32, dims 16 ks + 8 (l / 32) .. + 7 (read in the asm)
    const uint32_t qsr = la(lds + pr * PP_GROUP + PF_KB) + r32 * PF_QP + 16 * h;

    float m_run[2], l_run[2];
    asm volatile(PPL_ASM_MACROS R"ASM(
  .irp ks, 0,1,2,3,4,5,6,7,8,9,10,11,12,13,14,15
    ds_read_b128 v[4*\ks:4*\ks+3], %[qsr] offset:32*\ks
    ds_read_b128 v[64+4*\ks:67+4*\ks], %[qsr] offset:32*528+32*\ks
  .endr
  v_mov_b32 v236, 0xff800000
  v_mov_b32 v237, 0xff800000
  v_mov_b32 v238, 0
  v_mov_b32 v239, 0
  s_mov_b32 s85, 0
  s_mov_b64 s[92:93], 0
  s_sub_u32 s70, %[rowb], 1040
  s_subb_u32 s71, 0, 0
  s_sub_u32 s72, %[rowb], 1088
  s_subb_u32 s73, 0, 0
  s_waitcnt lgkmcnt(0)
  s_mov_b32 s84, 0
.Lppl_loop%=:
  s_cmp_eq_u32 s84, 0
  s_cbranch_scc0 .Lppl_topw%=
  s_waitcnt vmcnt(0)
.Lppl_topw%=:
  s_waitcnt vmcnt(8)
  s_barrier
  s_cmp_eq_u32 s85, 0
  s_cbranch_scc1 .Lppl_norescale%=
  s_waitcnt lgkmcnt(0)
  s_nop 7
  s_nop 7
  s_nop 7
  PPL_RESCALE_HEAD 0
  PPL_RESCALE_HEAD 1
  s_nop 3
  s_mov_b32 s85, 0
.Lppl_norescale%=:
  s_cmp_lt_u32 s84, %[n]
  s_cbranch_scc0 .Lppl_notile%=
  s_add_u32 s81, %[jb], s84
  s_lshl_b32 s82, s81, 5
  s_add_u32 s83, s82, 31
  s_cmp_gt_u32 s83, %[offt0]
  s_cselect_b32 s83, 1, 0
  s_bitcmp1_b32 s84, 0
  s_cselect_b32 s89, %[vc1], %[vc0]
  s_mov_b32 s97, 0
  s_mov_b32 s79, 0
  s_add_u32 s90, s84, 1
  s_cmp_lt_u32 s90, %[n]
  s_cbranch_scc0 .Lppl_nok%=
  s_bitcmp1_b32 s84, 0
  s_cselect_b32 s96, %[kc0], %[kc1]
  s_add_u32 s80, s81, 1
  s_mov_b32 s79, 1
  PPL_CSET %[klo], %[khi], s96, 1040, s94, s95, s97
.Lppl_nok%=:
  s_bitcmp1_b32 s84, 0
  s_cbranch_scc1 .Lppl_odd%=
  s_cmp_eq_u32 s84, 0
  s_cbranch_scc1 .Lppl_first%=
  PPL_TILE 1, 160, 176, %[kr0], %[vr1]
  s_branch .Lppl_next%=
.Lppl_first%=:
  PPL_TILE 0, 160, 176, %[kr0], %[vr1]
  s_branch .Lppl_next%=
.Lppl_odd%=:
  PPL_TILE 1, 176, 160, %[kr1], %[vr0]
  s_branch .Lppl_next%=
.Lppl_notile%=:
  s_cmp_eq_u32 s84, %[n]
  s_cbranch_scc0 .Lppl_idle%=
  s_cmp_eq_u32 s84, 0
  s_cbranch_scc1 .Lppl_idle%=
  s_bitcmp1_b32 s84, 0
  s_cbranch_scc0 .Lppl_lastodd%=
  PPL_LAST 160, %[vr0]
  s_branch .Lppl_next%=
.Lppl_lastodd%=:
  PPL_LAST 176, %[vr1]
  s_branch .Lppl_next%=
.Lppl_idle%=:
  s_barrier
.Lppl_next%=:
  s_add_u32 s84, s84, 1
  s_cmp_le_u32 s84, %[half]
  s_cbranch_scc1 .Lppl_loop%=
  s_waitcnt vmcnt(0) lgkmcnt(0)
  .purgem PPL_COPY
  .purgem PPL_CSET
  .purgem PPL_CROW
  .purgem PPL_KREAD
  .purgem PPL_VREAD
  .purgem PPL_PV
  .purgem PPL_PV1
  .purgem PPL_EXP2
  .purgem PPL_UPD1
  .purgem PPL_UPD2
  .purgem PPL_UPD3
  .purgem PPL_VY
  .purgem PPL_TILE
  .purgem PPL_LAST
  .purgem PPL_RESCALE_HEAD
)ASM"
                 : "+{a[0:15]}"(o[0][0]), "+{a[16:31]}"(o[0][1]), "+{a[32:47]}"(o[0][2]), "+{a[48:63]}"(o[0][3]),
                   "+{a[64:79]}"(o[0][4]), "+{a[80:95]}"(o[0][5]), "+{a[96:111]}"(o[0][6]), "+{a[112:127]}"(o[0][7]),
                   "+{a[128:143]}"(o[1][0]), "+{a[144:159]}"(o[1][1]), "+{a[160:175]}"(o[1][2]),
                   "+{a[176:191]}"(o[1][3]), "+{a[192:207]}"(o[1][4]), "+{a[208:223]}"(o[1][5]),
                   "+{a[224:239]}"(o[1][6]), "+{a[240:255]}"(o[1][7]), "={v236}"(m_run[0]), "={v237}"(m_run[1]),
                   "={v238}"(l_run[0]), "={v239}"(l_run[1])
                 : "{v224}"(k_lane), "{v225}"(v_lane), "{v226}"(lane_go), "{v227}"(limbase), "{v228}"(bcw),
                   "{v229}"(bcr), "{v230}"(h16), "{v231}"(r16), [qsr] "{v232}"(qsr), [n] "s"(un), [half] "s"(uhalf),
                   [jb] "s"(ujb), [nk] "s"(unk), [offt0] "s"(offt0), [klo] "s"(klo), [khi] "s"(khi), [vlo] "s"(vlo),
                   [vhi] "s"(vhi), [rowb] "s"(rowb), [pr8] "s"(pr8), [kr0] "s"(kr0), [kr1] "s"(kr1), [vr0] "s"(vr0),
                   [vr1] "s"(vr1), [kc0] "s"(kc0), [kc1] "s"(kc1), [vc0] "s"(vc0), [vc1] "s"(vc1)
                 : PP_CLOBBERS);
    // lane indices again, from the hardware (values computed before the loop would be held across it)
    const int el = __lane_id(), eh = el >> 5, er = el & 31;


    // Merge of the two key-range halves (group order), then 1/l, the gate and the stores. The merged rows are built in
    // LDS as [4 heads][32 tokens][256 dims] fp32 (pitch PP_OP, over the rings): each wave writes one head of its pair
    // there straight from the accumulation registers and merges its partner's dump of the other head into its own O in
    // place (O0 w0 / L + O1 w1 / L), then every wave stores whole rows (16 bytes per lane, gated) or rotates (token,
    // head pair) blocks.
    // The gate rows this wave stores (32 rows of 256, 16 bytes per lane; the rotation path takes rows by (token, head
    // pair) block) are requested now, so their latency passes under the merge.
    f4 gz[32];
    if (a.gate) {
#pragma unroll
        for (int i = 0; i < 32; i++) {
            // row i of this wave: (head kh 4 + hl, token tl); rotation: block m = i / 2 is (token tl, pair p), head 2p + i % 2
            const int k = a.signs ? w + 4 * (i >> 1) : w + 4 * i;
            const int tl = a.signs ? k >> 1 : k & 31;
            const int hl = a.signs ? 2 * (k & 1) + (i & 1) : k >> 5;
            const int t = min(t0 + tl, a.T - 1);
            gz[i] = *reinterpret_cast<const f4*>(a.gate + (int64_t)t * a.g_ts + (int64_t)(kh * 4 + hl) * a.g_hs + 4 * el);
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // every wave is done with the rings
    // each lane summed its own 16 keys of every tile; the row's sum takes the other lane half too (the swap runs on the
    // whole wave, outside any branch on the lane half)
    const float l_tot[2] = {sum_xhalf(l_run[0]), sum_xhalf(l_run[1])};
    if (eh == 0) {
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            ml_lds[w][hh][0][er] = m_run[hh];
            ml_lds[w][hh][1][er] = l_tot[hh];
        }
    }
    // this lane's element of register r of O tile (head 2 pr + hh, dims 32 dt ..): row 32 hh + 8 (r / 4) + r % 4 past
    // the lane's base (head 2 pr, token 4 (l / 32), dim l % 32), byte 128 dt. Wave (g, pr) hands head 2 pr + 1 - g of
    // its pair to its partner (same heads, other key half) and merges head 2 pr + g in place.
    const uint32_t obase = la(lds) + (uint32_t)((2 * pr * 32 + 4 * eh) * PP_OP + 4 * er);
    if (g == 0)
        pp_dump_o<1>(o, obase);
    else
        pp_dump_o<0>(o, obase);
    __syncthreads();
    {
        const int wp = w ^ 2, hm = g;  // partner wave; merged head of the pair
        if (eh == 0) {
            const float mo = ml_lds[w][hm][0][er], mp = ml_lds[wp][hm][0][er];
            const float lo = ml_lds[w][hm][1][er], lp = ml_lds[wp][hm][1][er];
            const float M = fmaxf(mo, mp);
            const float wo = mo == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mo - M);
            const float wq = mp == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mp - M);
            const float inv = 1.0f / (lo * wo + lp * wq);
            reinterpret_cast<float*>(bc_lds[w][hm][0])[er] = wo * inv;
            reinterpret_cast<float*>(bc_lds[w][hm][1])[er] = wq * inv;
        }
        // the factors are read back inside the merge, by this wave: its LDS writes are done first
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const uint32_t bc = la(&bc_lds[w][hm][0][0]) + 16 * eh;
        if (g == 0)
            pp_merge_o<0>(o, obase, bc);
        else
            pp_merge_o<1>(o, obase, bc);
    }
    __syncthreads();
    if (!a.signs) {
        // 128 rows (head, token) of 256 dims, 32 per wave
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const int k = w + 4 * i, hl = k >> 5, tl = k & 31, t = t0 + tl, hd = kh * 4 + hl;
            f4 y = *reinterpret_cast<const f4*>(lds + (hl * 32 + tl) * PP_OP + 16 * el);
            if (a.gate) {
#pragma unroll
                for (int e = 0; e < 4; e++) y[e] = gate_mul_fast(y[e], gz[i][e]);
            }
            if (t < a.T) *reinterpret_cast<f4*>(a.out + (int64_t)t * a.o_ts + (int64_t)hd * a.o_hs + 4 * el) = y;
        }
        return;
    }
    // rotation: (token tl, head pair p) blocks, 16 per wave; lane l holds dims 4l .. 4l+3 of heads 2p and 2p + 1
#pragma unroll
    for (int m = 0; m < 16; m++) {
        const int k = w + 4 * m, tl = k >> 1, p = k & 1, t = t0 + tl;
        if (t >= a.T) break;
        float v[8];
#pragma unroll
        for (int i2 = 0; i2 < 2; i2++) {
            const int hw = 2 * p + i2, hd = kh * 4 + hw;
            f4 y = *reinterpret_cast<const f4*>(lds + (hw * 32 + tl) * PP_OP + 16 * el);
            if (a.gate) {
#pragma unroll
                for (int e = 0; e < 4; e++) y[e] = gate_mul_fast(y[e], gz[2 * m + i2][e]);
            }
            y *= *reinterpret_cast<const f4*>(a.signs + (int64_t)hd * D + 4 * el);
#pragma unroll
            for (int c = 0; c < 4; c++) v[4 * i2 + c] = y[c];
        }
        fwht512_wave(v, el);
        float* o_ = a.out + (int64_t)t * a.o_ts + (int64_t)(kh * 4 + 2 * p) * a.o_hs;
#pragma unroll
        for (int i2 = 0; i2 < 2; i2++)
            *reinterpret_cast<f4*>(o_ + i2 * a.o_hs + 4 * el) =
                f4{v[4 * i2], v[4 * i2 + 1], v[4 * i2 + 2], v[4 * i2 + 3]} * INV_SQRT512;
    }
}

}  // namespace bn
