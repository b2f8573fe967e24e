// The key loop of prefill_pair_kernel as one block of gfx950 assembly with a fixed register map.
//
// Why assembly: a wave holds O of two heads (256 fp32 per lane, all accumulation registers), Q^T of both heads (128
// VGPRs), one S^T tile (32), two P tiles (32) and its LDS operand reads in flight: about 490 of the 512 registers a
// lane has at one wave per SIMD. Compiled, the loop spilled O or Q^T to scratch whatever the source shape; with every
// register placed by hand it fits with room to spare.
//
// Register map (per lane):
//   v[0:63]     Q^T of head 0: k-step ks (dims 16 ks + 8 (l / 32) .. +7, token l mod 32) in v[4 ks : 4 ks + 3]
//   v[64:127]   Q^T of head 1
//   v[128:143]  S^T of head 0 (keys 8 (r / 4) + 4 (l / 32) + r mod 4 of the tile, token l mod 32), v[144:159] head 1
//   v[160:175]  P buffer A, v[176:191] P buffer B: head hh, 16-key step kk in v[base + 8 hh + 4 kk : +3] (fp16 pairs)
//   v[192:223]  operand slots, 8 x 4 VGPRs: K operands in the S^T phase (6 reads ahead), V operands in the PV phase
//               (two ds_read_b64_tr_b16 each, 6 steps ahead); O's rescale factors at the loop top
//   v224 k_lane, v225 v_lane, v226 lane_go, v227 limbase, v228 bc write address, v229 bc read address, v230 16 (l / 32),
//   v231 16 (l mod 32), v232 Q staging address (inputs, not written)
//   v236, v237  running max m of heads 0, 1 (log2 domain); v238, v239 row sums l (outputs)
//   v240 K read address, v241 V read address; PV-phase softmax temporaries: v242-v245 exponent pairs, v246/v247 -m,
//   v248/v249 tile maxima, v250/v251 their lane-half swaps, v252/v253 scratch, v254/v255 rescale factors
//   a[0:255]    O: tile (head hh, dims 32 dt ..) in a[16 (8 hh + dt) : +15]
//   s80 key tile of a copy, s81 j, s82 j0, s83 diagonal flag, s84 i, s85 rescale pending, s[86:87] V row address, s88 V
//   row flag, s89 V M0 base, s[94:95] K row address, s96 K M0 base, s97 K row flag, s79 K copies issued this tile,
//   s[70:71] / s[72:73] rowb - 1040 / rowb - 1088 (64-bit row steps of the copies); s90, s91, s[92:93] copy
//   temporaries; in the PV phase s[92:93] rows whose max moved, s[94:97] lane masks
//
// Per tile i of the group (key tile j = jb + i): at the top, wait for this wave's K(j) copies (the 8 V copies of tile i - 1,
// issued after them, may still be in flight: vmcnt(8)) and a barrier (every wave's K(j) landed, every wave has left tile
// i - 1); rescale O if the previous tile moved a row's max; set up the copy of K(j + 1) into kst[(i + 1) mod 2]; then
//   S^T phase: S^T(j) = K(j) Q^T, 32 MFMAs, each K operand read (6 ahead) feeding both heads; the row sums take the
//     probabilities P(j - 1) meanwhile (one v_dot2 per k-step); K(j + 1)'s 8 row-pair copies go out at odd k-steps;
//   mid-tile: wait for V(j - 1) (copied in tile i - 1's PV phase) and a second barrier, then set up V(j)'s copy into
//     vst[i mod 2];
//   PV phase: O += P(j - 1) V(j - 1), 32 MFMAs, each transposed V operand read (6 ahead) feeding both heads; between
//     them the VALU masks S^T(j) (tiles across the diagonal only), takes the row maxima (v_max3, then the other lane
//     half by v_permlane32_swap), moves the running max when a row's tile max exceeds it by more than 8 (alpha =
//     2^(m - m'), l *= alpha, O *= alpha at the next tile), and writes P(j) = fp16(2^(S^T sc - m)) into the other P
//     buffer; V(j)'s 8 row-pair copies go out at odd steps.
// Copies are global_load_lds (no VGPRs); the instruction offset moves the global and the LDS address alike, so M0 is
// written once per four row pairs. The tile after the last one runs the last O += P V (after a wait and a barrier for
// its V tile). Every iteration passes exactly two barriers (the top one and the mid-tile, last-product or idle one), so
// groups with fewer tiles stay in step.
//
// Hazards the assembly keeps (the compiler does not see into it): XDL result -> VALU access 12 wait states (16 given
// after the S^T phase, 24 before the rescale); VALU write -> MFMA operand 2 (the P buffers are written a phase before
// their products; 4 after the rescale); trans (v_exp) result -> VALU read 1 (s_nop 0); VALU write -> permlane32_swap 2;
// VALU SGPR write -> SALU read (4 given); M0 write -> LDS DMA 1 (s_nop 0). Operand slots are reloaded two MFMA pairs
// after their last use. LDS and global results are waited for with lgkmcnt / vmcnt; every counter is drained at entry
// and exit.
#pragma once

namespace bn {

// clang-format off
#define PPL_ASM_MACROS R"ASM(
.macro PPL_COPY xlo, xhi, mb, pitch
  s_lshl_b32 s90, s80, 5
  s_add_u32 s91, s90, 32
  s_cmp_le_u32 s91, %[nk]
  s_cbranch_scc0 .Lppl_cpart\@
  s_add_u32 s91, s90, %[pr8]
  s_mul_i32 s92, s91, %[rowb]
  s_mul_hi_u32 s93, s91, %[rowb]
  s_add_u32 s92, s92, \xlo
  s_addc_u32 s93, s93, \xhi
  .irp r, 0,1,2,3,4,5,6,7
    s_add_u32 m0, \mb, (\r)*(\pitch)
    s_nop 0
    global_load_lds_dwordx4 v226, s[92:93]
    s_add_u32 s92, s92, %[rowb]
    s_addc_u32 s93, s93, 0
  .endr
  s_branch .Lppl_cdone\@
.Lppl_cpart\@:
  s_mul_i32 s92, s90, %[rowb]
  s_mul_hi_u32 s93, s90, %[rowb]
  s_add_u32 s92, s92, \xlo
  s_addc_u32 s93, s93, \xhi
  s_sub_u32 s91, %[nk], 1
  s_sub_u32 s91, s91, s90
  .irp r, 0,1,2,3,4,5,6,7
    s_add_u32 s90, %[pr8], \r
    v_add_u32 v[242+((\r)&1)], s90, v230
    v_min_i32 v[242+((\r)&1)], s91, v[242+((\r)&1)]
    v_mul_lo_u32 v[242+((\r)&1)], v[242+((\r)&1)], %[rowb]
    v_add_u32 v[242+((\r)&1)], v[242+((\r)&1)], v231
    s_add_u32 m0, \mb, (\r)*(\pitch)
    s_nop 0
    global_load_lds_dwordx4 v[242+((\r)&1)], s[92:93]
  .endr
.Lppl_cdone\@:
.endm

; Copy setup of a full tile for the S^T phase to issue row by row: if key tile s80 lies wholly inside the cache, the
; address of its first row pair in s[lo:lo+1] and flag = 1; otherwise the whole (clamped) copy is issued now, flag = 0.
.macro PPL_CSET xlo, xhi, mb, pitch, plo, phi, flag
  s_lshl_b32 s90, s80, 5
  s_add_u32 s91, s90, 32
  s_cmp_le_u32 s91, %[nk]
  s_cbranch_scc0 .Lppl_cset_part\@
  s_add_u32 s91, s90, %[pr8]
  s_mul_i32 \plo, s91, %[rowb]
  s_mul_hi_u32 \phi, s91, %[rowb]
  s_add_u32 \plo, \plo, \xlo
  s_addc_u32 \phi, \phi, \xhi
  s_mov_b32 \flag, 1
  s_branch .Lppl_cset_done\@
.Lppl_cset_part\@:
  PPL_COPY \xlo, \xhi, \mb, \pitch
  s_mov_b32 \flag, 0
.Lppl_cset_done\@:
.endm

; one row-pair copy of a tile set up by PPL_CSET (row pair r of the wave's eight, in order), if its flag says so. The
; instruction offset moves both addresses, so M0 is written once per four row pairs: row pair r lands at M0 + (r mod 4)
; pitch, and s[pair] steps by rowb - pitch (s[dlo:dhi], 64-bit) so that s[pair] + (r mod 4) pitch is its global row
.macro PPL_CROW r, mb, pitch, pair, plo, phi, flag, dlo, dhi
  s_cmp_eq_u32 \flag, 0
  s_cbranch_scc1 .Lppl_crow_skip\@
  .if ((\r) & 3) == 0
    s_add_u32 m0, \mb, (\r)*(\pitch)
    s_nop 0
  .endif
  global_load_lds_dwordx4 v226, s[\pair] offset:((\r)&3)*(\pitch)
  .if ((\r) & 3) == 3
    s_add_u32 \plo, \plo, %[rowb]
    s_addc_u32 \phi, \phi, 0
    s_add_u32 \plo, \plo, 3*(\pitch)
    s_addc_u32 \phi, \phi, 0
  .else
    s_add_u32 \plo, \plo, \dlo
    s_addc_u32 \phi, \phi, \dhi
  .endif
.Lppl_crow_skip\@:
.endm

.macro PPL_KREAD ks
  ds_read_b128 v[192+4*((\ks)&7):195+4*((\ks)&7)], v240 offset:32*(\ks)
.endm

.macro PPL_VREAD t
  ds_read_b64_tr_b16 v[192+4*((\t)&7):193+4*((\t)&7)], v241 offset:((\t)>>3)*512+64*((\t)&7)
  ds_read_b64_tr_b16 v[194+4*((\t)&7):195+4*((\t)&7)], v241 offset:((\t)>>3)*512+64*((\t)&7)+8704
.endm

.macro PPL_PV t, pp
  v_mfma_f32_32x32x16_f16 a[16*((\t)&7):16*((\t)&7)+15], v[\pp+4*((\t)>>3):\pp+4*((\t)>>3)+3], v[192+4*((\t)&7):195+4*((\t)&7)], a[16*((\t)&7):16*((\t)&7)+15]
.endm
.macro PPL_PV1 t, pp
  v_mfma_f32_32x32x16_f16 a[128+16*((\t)&7):128+16*((\t)&7)+15], v[\pp+8+4*((\t)>>3):\pp+8+4*((\t)>>3)+3], v[192+4*((\t)&7):195+4*((\t)&7)], a[128+16*((\t)&7):128+16*((\t)&7)+15]
.endm

; one probability pair: head hh, registers 2 p2, 2 p2 + 1 of its S^T tile -> one fp16 pair of P buffer pc
.macro PPL_EXP2 hh, p2, pc, ta, tb
  v_fmamk_f32 v\ta, v[128+16*(\hh)+2*(\p2)], 0x3db8aa3b, v[246+(\hh)]
  v_fmamk_f32 v\tb, v[129+16*(\hh)+2*(\p2)], 0x3db8aa3b, v[246+(\hh)]
  v_exp_f32 v\ta, v\ta
  v_exp_f32 v\tb, v\tb
  s_nop 0
  v_cvt_pk_f16_f32 v[\pc+8*(\hh)+(\p2)], v\ta, v\tb
.endm

; running max of head hh (tile max in v[248+hh] already scaled): m, l, alpha (kept in v[254+hh]), -m (or 0) in v[246+hh]
.macro PPL_UPD1 hh
  v_add_f32 v252, 0x41000000, v[236+(\hh)]
  v_cmp_gt_f32_e64 s[94:95], v[248+(\hh)], v252
  v_sub_f32 v253, v[236+(\hh)], v[248+(\hh)]
  v_exp_f32 v253, v253
.endm
.macro PPL_UPD2 hh
  s_nop 0
  v_cmp_class_f32_e64 s[96:97], v[236+(\hh)], 4
  v_cndmask_b32_e64 v[254+(\hh)], 1.0, v253, s[94:95]
  v_cndmask_b32_e64 v[236+(\hh)], v[236+(\hh)], v[248+(\hh)], s[94:95]
  v_mul_f32 v[238+(\hh)], v[238+(\hh)], v[254+(\hh)]
.endm
.macro PPL_UPD3 hh
  s_nop 4
  s_andn2_b64 s[96:97], s[94:95], s[96:97]
  s_or_b64 s[92:93], s[92:93], s[96:97]
  v_cmp_class_f32_e64 s[94:95], v[236+(\hh)], 4
  v_cndmask_b32_e64 v[246+(\hh)], -v[236+(\hh)], 0, s[94:95]
.endm

; softmax work of the PV phase, slot k (two slots per PV step, one after each MFMA); pc: P buffer written
.macro PPL_VY k, pc
  .if \k == 0
    v_max3_f32 v248, v128, v129, v130
    v_max3_f32 v248, v248, v131, v132
    v_max3_f32 v248, v248, v133, v134
    v_max3_f32 v248, v248, v135, v136
  .elseif \k == 1
    v_max3_f32 v248, v248, v137, v138
    v_max3_f32 v248, v248, v139, v140
    v_max3_f32 v248, v248, v141, v142
    v_max_f32 v248, v248, v143
  .elseif \k == 2
    v_max3_f32 v249, v144, v145, v146
    v_max3_f32 v249, v249, v147, v148
    v_max3_f32 v249, v249, v149, v150
    v_max3_f32 v249, v249, v151, v152
  .elseif \k == 3
    v_max3_f32 v249, v249, v153, v154
    v_max3_f32 v249, v249, v155, v156
    v_max3_f32 v249, v249, v157, v158
    v_max_f32 v249, v249, v159
  .elseif \k == 4
    v_mov_b32 v250, v248
    v_mov_b32 v251, v249
    s_nop 1
    v_permlane32_swap_b32 v248, v250
    v_permlane32_swap_b32 v249, v251
  .elseif \k == 5
    v_max_f32 v248, v248, v250
    v_max_f32 v249, v249, v251
    v_mul_f32 v248, 0x3db8aa3b, v248
    v_mul_f32 v249, 0x3db8aa3b, v249
  .elseif \k == 6
    PPL_UPD1 0
  .elseif \k == 7
    PPL_UPD2 0
  .elseif \k == 8
    PPL_UPD3 0
  .elseif \k == 9
    PPL_UPD1 1
  .elseif \k == 10
    PPL_UPD2 1
    PPL_EXP2 0, 0, \pc, 242, 243
  .elseif \k == 11
    PPL_UPD3 1
    s_nop 4
    s_cmp_lg_u64 s[92:93], 0
    s_cselect_b32 s85, 1, 0
    PPL_EXP2 0, 1, \pc, 244, 245
  .elseif \k == 12
    PPL_EXP2 0, 2, \pc, 242, 243
  .elseif \k == 13
    PPL_EXP2 0, 3, \pc, 244, 245
  .elseif \k == 14
    PPL_EXP2 0, 4, \pc, 242, 243
  .elseif \k == 15
    PPL_EXP2 0, 5, \pc, 244, 245
  .elseif \k == 17
    PPL_EXP2 0, 6, \pc, 242, 243
  .elseif \k == 18
    PPL_EXP2 0, 7, \pc, 244, 245
  .elseif \k == 19
    PPL_EXP2 1, 0, \pc, 242, 243
  .elseif \k == 20
    PPL_EXP2 1, 1, \pc, 244, 245
  .elseif \k == 22
    PPL_EXP2 1, 2, \pc, 242, 243
  .elseif \k == 23
    PPL_EXP2 1, 3, \pc, 244, 245
  .elseif \k == 24
    PPL_EXP2 1, 4, \pc, 242, 243
  .elseif \k == 26
    PPL_EXP2 1, 5, \pc, 244, 245
  .elseif \k == 27
    PPL_EXP2 1, 6, \pc, 242, 243
  .elseif \k == 28
    PPL_EXP2 1, 7, \pc, 244, 245
  .elseif \k == 31
    ds_write_b32 v228, v254
    ds_write_b32 v228, v255 offset:128
  .endif
.endm

; one tile: S^T(j) from the K stage at LDS address kr; with pv, O += P(j - 1) V(j - 1) from P buffer pp and the V stage
; at vr; P(j) into P buffer pc
.macro PPL_TILE pv, pc, pp, kr, vr
  v_add_u32 v240, \kr, v224
  .irp ks, 0,1,2,3,4,5
    PPL_KREAD \ks
  .endr
  .irp ks, 0,1,2,3,4,5,6,7,8,9,10,11,12,13,14,15
    .if \ks + 6 <= 15
      PPL_KREAD \ks+6
      s_waitcnt lgkmcnt(6)
    .else
      s_waitcnt lgkmcnt(15-\ks)
    .endif
    .if \ks == 0
      v_mfma_f32_32x32x16_f16 v[128:143], v[192:195], v[0:3], 0
    .else
      v_mfma_f32_32x32x16_f16 v[128:143], v[192+4*((\ks)&7):195+4*((\ks)&7)], v[4*\ks:4*\ks+3], v[128:143]
    .endif
    .if \pv
      .if \ks < 8
        v_dot2c_f32_f16 v238, 0x3c003c00, v[\pp+\ks]
      .else
        v_dot2c_f32_f16 v239, 0x3c003c00, v[\pp+\ks]
      .endif
    .endif
    .if \ks == 0
      v_mfma_f32_32x32x16_f16 v[144:159], v[192:195], v[64:67], 0
    .else
      v_mfma_f32_32x32x16_f16 v[144:159], v[192+4*((\ks)&7):195+4*((\ks)&7)], v[64+4*\ks:67+4*\ks], v[144:159]
    .endif
    .if (\ks & 1)
      PPL_CROW (\ks)>>1, s96, 1040, 94:95, s94, s95, s97, s70, s71
    .endif
  .endr
  s_nop 7
  s_nop 7
  s_cmp_eq_u32 s79, 0
  s_cbranch_scc1 .Lppl_mid0\@
  s_waitcnt vmcnt(8)
  s_branch .Lppl_midw\@
.Lppl_mid0\@:
  s_waitcnt vmcnt(0)
.Lppl_midw\@:
  s_barrier
  s_mov_b32 s80, s81
  PPL_CSET %[vlo], %[vhi], s89, 1088, s86, s87, s88
  .if \pv
    v_add_u32 v241, \vr, v225
    .irp t, 0,1,2,3,4,5
      PPL_VREAD \t
    .endr
  .endif
  s_cmp_eq_u32 s83, 0
  s_cbranch_scc1 .Lppl_nomask\@
  v_subrev_u32 v252, s82, v227
  v_mov_b32 v253, 0xff800000
  .irp r, 0,1,2,3,4,5,6,7,8,9,10,11,12,13,14,15
    v_cmp_le_i32 vcc, 8*((\r)>>2)+((\r)&3), v252
    v_cndmask_b32 v[128+\r], v253, v[128+\r], vcc
    v_cndmask_b32 v[144+\r], v253, v[144+\r], vcc
  .endr
.Lppl_nomask\@:
  s_mov_b64 s[92:93], 0
  .if \pv
    .irp t, 0,1,2,3,4,5,6,7,8,9,10,11,12,13,14,15
      .if \t + 6 <= 15
        PPL_VREAD \t+6
        s_waitcnt lgkmcnt(12)
      .else
        s_waitcnt lgkmcnt(2*(15-\t))
      .endif
      PPL_PV \t, \pp
      PPL_VY 2*\t, \pc
      PPL_PV1 \t, \pp
      .if (\t & 1)
        PPL_CROW (\t)>>1, s89, 1088, 86:87, s86, s87, s88, s72, s73
      .endif
      PPL_VY 2*\t+1, \pc
    .endr
  .else
    .irp k, 0,1,2,3,4,5,6,7,8,9,10,11,12,13,14,15,16,17,18,19,20,21,22,23,24,25,26,27,28,29,30,31
      .if (\k & 3) == 3
        PPL_CROW (\k)>>2, s89, 1088, 86:87, s86, s87, s88, s72, s73
      .endif
      PPL_VY \k, \pc
    .endr
  .endif
.endm

; O += P V of the group's last tile (P buffer pp, V stage at vr), after its row sums
.macro PPL_LAST pp, vr
  s_waitcnt vmcnt(0) lgkmcnt(0)
  s_barrier
  .irp k, 0,1,2,3,4,5,6,7
    v_dot2c_f32_f16 v238, 0x3c003c00, v[\pp+\k]
    v_dot2c_f32_f16 v239, 0x3c003c00, v[\pp+8+\k]
  .endr
  v_add_u32 v241, \vr, v225
  .irp t, 0,1,2,3,4,5
    PPL_VREAD \t
  .endr
  .irp t, 0,1,2,3,4,5,6,7,8,9,10,11,12,13,14,15
    .if \t + 6 <= 15
      PPL_VREAD \t+6
      s_waitcnt lgkmcnt(12)
    .else
      s_waitcnt lgkmcnt(2*(15-\t))
    .endif
    PPL_PV \t, \pp
    PPL_PV1 \t, \pp
  .endr
.endm

; O *= alpha per row, alphas of head hh from the wave's broadcast slots (16 per lane: rows 8 q + 4 (l / 32) + e)
.macro PPL_RESCALE_HEAD hh
  ds_read_b128 v[192:195], v229 offset:128*(\hh)
  ds_read_b128 v[196:199], v229 offset:128*(\hh)+32
  ds_read_b128 v[200:203], v229 offset:128*(\hh)+64
  ds_read_b128 v[204:207], v229 offset:128*(\hh)+96
  s_waitcnt lgkmcnt(0)
  .irp k, 0,1,2,3,4,5,6,7
    .irp r, 0,1,2,3,4,5,6,7,8,9,10,11,12,13,14,15
      v_accvgpr_read_b32 v[242+((\r)&3)], a[16*(8*(\hh)+\k)+\r]
      v_mul_f32 v[242+((\r)&3)], v[242+((\r)&3)], v[192+\r]
      v_accvgpr_write_b32 a[16*(8*(\hh)+\k)+\r], v[242+((\r)&3)]
    .endr
  .endr
.endm
)ASM"
// clang-format on

}  // namespace bn
