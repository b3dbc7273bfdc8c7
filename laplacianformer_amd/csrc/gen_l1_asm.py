#!/usr/bin/env python3
"""Generator of the hand-scheduled gfx950 inner loops of the L1 backward.

Writes ``l1_asm_gen.h``: one ``__device__`` function per (element type, key
count M) holding a single ``asm volatile`` block. The block is the whole row
loop of one wave of the column-split backward (see ``laplace_bwd2.hip``):
staging of the grad rows into LDS, the per-triple arithmetic and the
grad_query stores. It is generated rather than written by hand because its
value lies in the register map:

* every VALU instruction reads VGPR operands only (an SGPR operand halves the
  issue rate on gfx950);
* ``v_fmac_f32`` is issued with src0 and the accumulator in different VGPR
  banks (bank = register number mod 4; a clash halves the issue rate). Each
  product has two candidate src0 registers in different banks (the grad value
  and the step value), and the generator picks the one whose bank differs
  from the accumulator's;
* hazards the hardware does not interlock are covered explicitly (``s_nop``
  before DPP and ``v_permlane32_swap`` reads of just-written VGPRs): the
  compiler does not insert wait states inside inline asm.

The arithmetic per (row i, key column j, channel c), with T() the
order-preserving map of a 16-bit float pattern onto the fp32 values
2^22 + 2^14 + t/2 (t = signed magnitude of the pattern, so +0 and -0 coincide):

    y   = clamp(T(q[i,c]) + (0.5 - T(k[c,j])))      # (sgn(q - k) + 1) / 2, exact
    dq += (2 g[i,j]) * y                            # grad_query: sum_j 2g y - sum_j g
    dk[j] += (2 g[i,j]) * y                         # grad_key:  sum_i g - sum_i 2g y

Run as ``python gen_l1_asm.py <out.h>`` (the build does this).
"""
from __future__ import annotations

import sys

RB = 8            # grad rows per staged batch
LANES = 64


class Regs:
    """Top-down VGPR allocator for the asm block's private registers."""

    def __init__(self, top=256):
        self.next = top

    def take(self, n, align=1, bank=None):
        base = self.next - n
        while base % align != 0 or (bank is not None and base % 4 != bank):
            base -= 1
        self.next = base
        return base


def variant(dtype, M, DQ=True, DK=True):
    """Returns (name, C++ source, info) of the backward row-loop block for key count M.

    DQ / DK select the grad_query and grad_key halves of the work: without DK
    there are no grad_key accumulators or column sums, without DQ no row sums,
    grad_query accumulation or stores."""
    assert DQ or DK
    JC = (M + 1) // 2                 # key columns per lane half (half 1 may hold one pad column)
    EPL = (M + 7) // 8                # staged grad elements per lane (8 lanes per row)
    assert M % EPL == 0, "every staging lane holds whole runs of one row"
    XV = M // EPL                     # staging lanes per row that hold real columns
    HP = ((JC + 1 + 3) // 4) * 4      # LDS slots per half row: JC columns, the row sum, padding
    NG = HP // 4                      # 16-byte groups per half row
    PITCH = 2 * HP                    # floats per staged row
    RSLOT = JC                        # slot of the row sum in each half
    bf16 = dtype == "bf16"

    # Register banks (number mod 4) measured fastest for this loop at two waves per
    # SIMD: the step values Y at the parity opposite to the grad values G (a src0 /
    # src1 pair of equal parity costs a co-issue slot), the two grad_query
    # accumulators in banks 1 and 2, grad_key sums starting in bank 1.
    r = Regs()
    KK = r.take(4 * ((2 * JC + 3) // 4), align=4)   # 0.5 - T(k): [c][j] packed, read as b128 groups
    DK = r.take(2 * JC, bank=1) if DK else None       # grad_key accumulators [c][j]
    G = r.take(16, align=4)                           # grad ring: 4 slots of 4 (bank k for element k)
    Y = r.take(8, bank=3)                             # step values [c][k] (bank (k + 3) mod 4)
    DQR = [r.take(1, bank=1), r.take(1, bank=2)] if DQ else None   # grad_query accumulators [c]
    TQ = r.take(2 * RB, bank=1)                       # T(q) of the batch rows [row][c]
    QRAW = r.take(RB)                                 # raw query patterns of the next batch
    GRAW = r.take(EPL)                                # raw grad elements of the next batch
    CS = r.take(EPL) if DK else None                  # column sums of 2g (this lane's staging columns)
    RDA = r.take(1)       # LDS read base of the lane's half (slot base + h * HP * 4)
    VQ = r.take(1)        # byte offset of the lane's channel in a query / grad_query row
    GOFF = r.take(1)      # staging byte offset of the lane's first element in a full batch
    GOFFT = r.take(1)     # the same for the final partial batch (rows clamped to the last one)
    ST = r.take(EPL)      # LDS byte addresses of the lane's staged elements
    RS = r.take(1)        # LDS byte address for the lane's row-sum write (or a scratch slot)
    VX = r.take(1)        # 1.0 if the lane's staging columns are real, else 0.0
    VR = r.take(1)        # row validity of the staged batch for the column sums (1.0 / 0.0)
    VRT = r.take(1)       # row validity in the final partial batch
    T0 = r.take(4)        # temporaries
    lo = r.next
    nmine = 256 - lo

    # SGPRs (clobbered): pointers and counters.
    S = 72
    SG, SQ, SD = S, S + 2, S + 4          # 64-bit: next g batch, next q batch row, current dq row
    SQS, SBS = S + 6, S + 7               # q/dq row stride (bytes), g batch stride (bytes)
    SNB, STL = S + 8, S + 9               # full batches left to load, rows of the final batch (0..7)
    SROWS = S + 10                        # rows of the batch being computed
    SLD = S + 11                          # kind of the batch loaded next: 0 none, 1 full, 2 final
    STMP = S + 12                         # 64-bit temporary
    SGT = S + 14                          # 64-bit: g pointer of the final partial batch
    SQT = S + 16                          # 64-bit: q pointer of the final partial batch
    SCNT = S + 18                         # batches left to compute
    STN = S + 19                          # rows of the final partial batch (constant)
    SPR = S + 20                          # priority phase of this wave (flips every batch)
    SREG_HI = S + 20

    L = []
    add = L.append

    def grp_cols(g):
        return [j for j in range(4 * g, min(JC, 4 * g + 4))]

    def fmac(acc, gk, yk):
        """v_fmac acc += gk * yk with src0 in a bank different from acc's."""
        if gk % 4 != acc % 4:
            return f"v_fmac_f32 v{acc}, v{gk}, v{yk}"
        return f"v_fmac_f32 v{acc}, v{yk}, v{gk}"

    def fmul(dst, gk, yk):
        return f"v_mul_f32 v{dst}, v{gk}, v{yk}"

    # ---- entry: inputs into private registers --------------------------------
    add("s_waitcnt vmcnt(0) lgkmcnt(0)")
    add(f"s_mov_b64 s[{SG}:{SG+1}], %[g]")
    add(f"s_mov_b64 s[{SQ}:{SQ+1}], %[q]")
    add(f"s_mov_b64 s[{SD}:{SD+1}], %[dq]")
    add(f"s_mov_b32 s{SQS}, %[qs]")
    add(f"s_mov_b32 s{SBS}, {RB * M * 2}")
    add(f"s_mov_b32 s{SNB}, %[nb]")
    add(f"s_mov_b32 s{STL}, %[tail]")
    add(f"s_mov_b32 s{STN}, %[tail]")
    add(f"s_mov_b32 s{SPR}, %[wpar]")
    add(f"s_mov_b64 s[{SGT}:{SGT+1}], %[gt]")
    add(f"s_mov_b64 s[{SQT}:{SQT+1}], %[qt]")
    for reg, op in ((RDA, "rda"), (VQ, "vq"), (GOFF, "goff"), (GOFFT, "gofft"), (RS, "rs"), (VX, "vx"),
                    (VRT, "vrt")):
        add(f"v_mov_b32 v{reg}, %[{op}]")
    for e in range(EPL):
        add(f"v_mov_b32 v{ST + e}, %[st{e}]")
    # Key terms from the workgroup table (lane-private 16-byte groups).
    for i in range((2 * JC + 3) // 4):
        add(f"ds_read_b128 v[{KK + 4*i}:{KK + 4*i + 3}], %[kka] offset:{i * LANES * 16}")
    if DK:
        for j in range(2 * JC):
            add(f"v_mov_b32 v{DK + j}, 0")
        for e in range(EPL):
            add(f"v_mov_b32 v{CS + e}, 0")
    add(f"s_add_u32 s{SCNT}, s{SNB}, 0")
    add(f"s_cmp_lg_u32 s{STL}, 0")
    add(f"s_addc_u32 s{SCNT}, s{SCNT}, 0")   # batches to compute = full + (tail != 0)

    # ---- loads of one batch (kind in SLD): EPL grad elements + RB query patterns --------
    def emit_loads(lbl):
        add(f"s_cmp_eq_u32 s{SLD}, 0")
        add(f"s_cbranch_scc1 {lbl}_none")
        add(f"s_cmp_eq_u32 s{SLD}, 2")
        add(f"s_cbranch_scc1 {lbl}_tail")
        for e in range(EPL):
            add(f"global_load_ushort v{GRAW + e}, v{GOFF}, s[{SG}:{SG+1}] offset:{2 * e}")
        add(f"s_mov_b64 s[{STMP}:{STMP+1}], s[{SQ}:{SQ+1}]")
        for rr in range(RB):
            add(f"global_load_ushort v{QRAW + rr}, v{VQ}, s[{STMP}:{STMP+1}]")
            if rr + 1 < RB:
                add(f"s_add_u32 s{STMP}, s{STMP}, s{SQS}")
                add(f"s_addc_u32 s{STMP+1}, s{STMP+1}, 0")
        add(f"s_add_u32 s{SG}, s{SG}, s{SBS}")
        add(f"s_addc_u32 s{SG+1}, s{SG+1}, 0")
        add(f"s_add_u32 s{SQ}, s{STMP}, s{SQS}")
        add(f"s_addc_u32 s{SQ+1}, s{STMP+1}, 0")
        add(f"s_branch {lbl}_none")
        add(f"{lbl}_tail:")
        for e in range(EPL):
            add(f"global_load_ushort v{GRAW + e}, v{GOFFT}, s[{SGT}:{SGT+1}] offset:{2 * e}")
        add(f"s_mov_b64 s[{STMP}:{STMP+1}], s[{SQT}:{SQT+1}]")
        for rr in range(RB):
            # Rows past the final batch's end are not loaded (their values are never used).
            add(f"s_cmp_le_u32 s{STN}, {rr}")
            add(f"s_cbranch_scc1 {lbl}_none")
            add(f"global_load_ushort v{QRAW + rr}, v{VQ}, s[{STMP}:{STMP+1}]")
            add(f"s_add_u32 s{STMP}, s{STMP}, s{SQS}")
            add(f"s_addc_u32 s{STMP+1}, s{STMP+1}, 0")
        add(f"{lbl}_none:")

    # Kind of the next batch to load (SLD): 1 full, 2 the final partial one, 0 none.
    def next_kind(lbl):
        add(f"s_mov_b32 s{SLD}, 0")
        add(f"s_cmp_eq_u32 s{SNB}, 0")
        add(f"s_cbranch_scc1 {lbl}_t")
        add(f"s_mov_b32 s{SLD}, 1")
        add(f"s_sub_u32 s{SNB}, s{SNB}, 1")
        add(f"s_branch {lbl}_d")
        add(f"{lbl}_t:")
        add(f"s_cmp_eq_u32 s{STL}, 0")
        add(f"s_cbranch_scc1 {lbl}_d")
        add(f"s_mov_b32 s{SLD}, 2")
        add(f"s_mov_b32 s{STL}, 0")
        add(f"{lbl}_d:")

    # Staging of the loaded batch into LDS (2g as fp32), column sums, row sums, T(q).
    def emit_stage(vmc):
        # The batch's loads are older than the vmc grad_query stores issued since.
        add(f"s_waitcnt vmcnt({vmc})")
        for e in range(EPL):
            if bf16:
                add(f"v_lshlrev_b32 v{GRAW + e}, 16, v{GRAW + e}")
            else:
                add(f"v_cvt_f32_f16 v{GRAW + e}, v{GRAW + e}")
        for e in range(EPL):
            add(f"v_add_f32 v{GRAW + e}, v{GRAW + e}, v{GRAW + e}")
        for e in range(EPL):
            add(f"ds_write_b32 v{ST + e}, v{GRAW + e}")
        if DK:
            for e in range(EPL):
                add(f"v_fmac_f32 v{CS + e}, v{GRAW + e}, v{VR}")
        if DQ:
            # Row sum: this lane's run, then the 8 lanes of the row (DPP within 16-lane rows).
            add(f"v_add_f32 v{T0}, v{GRAW}, v{GRAW + 1}" if EPL > 1 else f"v_mov_b32 v{T0}, v{GRAW}")
            for e in range(2, EPL):
                add(f"v_add_f32 v{T0}, v{T0}, v{GRAW + e}")
            add(f"v_mul_f32 v{T0}, v{T0}, v{VX}")
            add("s_nop 1")
            add(f"v_add_f32_dpp v{T0 + 1}, v{T0}, v{T0} quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf")
            add("s_nop 1")
            add(f"v_add_f32_dpp v{T0 + 2}, v{T0 + 1}, v{T0 + 1} quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf")
            add("s_nop 1")
            add(f"v_add_f32_dpp v{T0 + 3}, v{T0 + 2}, v{T0 + 2} row_ror:12 row_mask:0xf bank_mask:0xf")
            add(f"v_mul_f32 v{T0 + 3}, 0.5, v{T0 + 3}")
            add(f"ds_write_b32 v{RS}, v{T0 + 3}")
        # T(q): t = signed magnitude of the pattern; T = as_float(0x4a808000 + t).
        for rr in range(RB):
            x = QRAW + rr
            add(f"v_and_b32 v{T0}, 0x7fff, v{x}")
            add(f"v_bfe_i32 v{T0 + 1}, v{x}, 15, 1")
            add(f"v_sub_u32 v{T0 + 2}, 0x4a808000, v{T0 + 1}")
            add(f"v_xad_u32 v{TQ + 2*rr}, v{T0}, v{T0 + 1}, v{T0 + 2}")
            add(f"v_mov_b32 v{TQ + 2*rr + 1}, v{TQ + 2*rr}")
        add("s_nop 4")
        # Lanes 0-31 computed T for channel 2p, lanes 32-63 for 2p + 1; after the
        # swap every lane holds both, [row][0] = channel 2p, [row][1] = 2p + 1.
        for rr in range(RB):
            add(f"v_permlane32_swap_b32 v{TQ + 2*rr}, v{TQ + 2*rr + 1}")
        add("s_nop 1")

    # ---- prologue: batch 0 (its raw elements were loaded by the caller) ----------
    add(f"v_mov_b32 v{VR}, 1.0")
    next_kind("NK0_%=")
    for e in range(EPL):
        add(f"v_mov_b32 v{GRAW + e}, %[g0_{e}]")
    for rr in range(RB):
        add(f"v_mov_b32 v{QRAW + rr}, %[q0_{rr}]")
    # A preloaded full batch moves the load pointers on, as emit_loads does.
    add(f"s_cmp_eq_u32 s{SLD}, 1")
    add("s_cbranch_scc0 PA_%=")
    add(f"s_add_u32 s{SG}, s{SG}, s{SBS}")
    add(f"s_addc_u32 s{SG+1}, s{SG+1}, 0")
    add(f"s_mul_i32 s{STMP}, s{SQS}, {RB}")
    add(f"s_add_u32 s{SQ}, s{SQ}, s{STMP}")
    add(f"s_addc_u32 s{SQ+1}, s{SQ+1}, 0")
    add("PA_%=:")
    add(f"s_cmp_eq_u32 s{SLD}, 2")
    add(f"s_cbranch_scc0 P0_%=_full")
    add(f"v_mov_b32 v{VR}, v{VRT}")
    add(f"s_mov_b32 s{SROWS}, s{STN}")
    add(f"s_branch P0_%=_st")
    add(f"P0_%=_full:")
    add(f"s_mov_b32 s{SROWS}, {RB}")
    add(f"P0_%=_st:")
    add("s_waitcnt lgkmcnt(0)")
    emit_stage(0)
    next_kind("NK1_%=")
    emit_loads("LD1_%=")

    # ---- batch loop ------------------------------------------------------------
    add("BL_%=:")
    # The two waves sharing a SIMD take turns at the higher issue priority, one
    # batch each, so that neither runs ahead and finishes alone.
    add(f"s_xor_b32 s{SPR}, s{SPR}, 1")
    add(f"s_cmp_eq_u32 s{SPR}, 0")
    add("s_cbranch_scc1 PR_%=_lo")
    add("s_setprio 2")
    add("s_branch PR_%=_d")
    add("PR_%=_lo:")
    add("s_setprio 0")
    add("PR_%=_d:")
    add("s_waitcnt lgkmcnt(0)")
    nstream = RB * NG
    ring = 4
    ahead = 3

    def pos_addr(p):
        rr, g = divmod(p, NG)
        return (rr * PITCH + 4 * g) * 4

    for p in range(ahead):
        add(f"ds_read_b128 v[{G + 4*(p % ring)}:{G + 4*(p % ring) + 3}], v{RDA} offset:{pos_addr(p)}")
    for rr in range(RB):
        if rr > 0:
            add(f"s_cmp_le_u32 s{SROWS}, {rr}")
            add("s_cbranch_scc1 BE_%=")
        for g in range(NG):
            p = rr * NG + g
            pn = p + ahead
            add(f"ds_read_b128 v[{G + 4*(pn % ring)}:{G + 4*(pn % ring) + 3}], v{RDA} offset:{pos_addr(pn)}")
            add(f"s_waitcnt lgkmcnt({ahead})")
            gs = G + 4 * (p % ring)
            cols = grp_cols(g)
            for c in range(2):
                for k, j in enumerate(cols):
                    add(f"v_add_f32_e64 v{Y + 4*c + k}, v{TQ + 2*rr + c}, v{KK + c*JC + j} clamp")
            for k, j in enumerate(cols):
                for c in range(2):
                    if DQ:
                        if j == 0:
                            add(fmul(DQR[c], gs + k, Y + 4*c + k))
                        else:
                            add(fmac(DQR[c], gs + k, Y + 4*c + k))
                    if DK:
                        add(fmac(DK + c*JC + j, gs + k, Y + 4*c + k))
        if not DQ:
            continue
        # Row finalize: halves combined, row sum subtracted, rounded, stored.
        rg = G + 4 * ((rr * NG + NG - 1) % ring) + (RSLOT % 4)
        assert RSLOT // 4 == NG - 1
        add("s_nop 4")
        add(f"v_permlane32_swap_b32 v{DQR[0]}, v{DQR[1]}")
        add("s_nop 1")
        add(f"v_add_f32 v{T0}, v{DQR[0]}, v{DQR[1]}")
        add(f"v_sub_f32 v{T0}, v{T0}, v{rg}")
        if bf16:
            add(f"v_cvt_pk_bf16_f32 v{T0}, v{T0}, v{T0}")
        else:
            add(f"v_cvt_f16_f32 v{T0}, v{T0}")
        add(f"global_store_short v{VQ}, v{T0}, s[{SD}:{SD+1}]")
        add(f"s_add_u32 s{SD}, s{SD}, s{SQS}")
        add(f"s_addc_u32 s{SD+1}, s{SD+1}, 0")
    add("BE_%=:")
    add(f"s_sub_u32 s{SCNT}, s{SCNT}, 1")
    add(f"s_cmp_eq_u32 s{SCNT}, 0")
    add("s_cbranch_scc1 BX_%=")
    # Stage the batch whose loads were issued during this one, then load the next.
    add("s_waitcnt lgkmcnt(0)")
    add(f"s_cmp_eq_u32 s{SLD}, 2")
    add(f"s_cbranch_scc0 BS_%=_full")
    add(f"v_mov_b32 v{VR}, v{VRT}")
    add(f"s_mov_b32 s{SROWS}, s{STN}")
    add(f"s_branch BS_%=_st")
    add(f"BS_%=_full:")
    add(f"s_mov_b32 s{SROWS}, {RB}")
    add(f"BS_%=_st:")
    emit_stage(RB if DQ else 0)
    next_kind("NKN_%=")
    emit_loads("LDN_%=")
    add("s_branch BL_%=")
    add("BX_%=:")
    add("s_setprio 0")
    add("s_waitcnt vmcnt(0) lgkmcnt(0)")
    if DK:
        for j in range(2 * JC):
            add(f"v_mov_b32 %[dk{j}], v{DK + j}")
        for e in range(EPL):
            add(f"v_mov_b32 %[cs{e}], v{CS + e}")

    # ---- C++ wrapper -----------------------------------------------------------
    name = f"bwd2_rows_{dtype}_m{M}_{'q' if DQ else ''}{'k' if DK else ''}"
    asm = "\n".join("      \"" + s + "\\n\"" for s in L)
    outs = ", ".join([f"[dk{j}] \"=v\"(dk[{j}])" for j in range(2 * JC)] +
                     [f"[cs{e}] \"=v\"(cs[{e}])" for e in range(EPL)]) if DK else ""
    ins = ", ".join([
        "[g] \"s\"(g)", "[q] \"s\"(q)", "[dq] \"s\"(dq)", "[qs] \"s\"(qstride)", "[nb] \"s\"(nfull)",
        "[tail] \"s\"(tail)", "[gt] \"s\"(gtail)", "[qt] \"s\"(qtail)",
        "[rda] \"v\"(rda)", "[vq] \"v\"(vq)", "[goff] \"v\"(goff)", "[gofft] \"v\"(gofft)", "[rs] \"v\"(rs)",
        "[vx] \"v\"(vx)", "[vrt] \"v\"(vrt)", "[kka] \"v\"(kka)", "[wpar] \"s\"(wpar)"] +
        [f"[st{e}] \"v\"(st[{e}])" for e in range(EPL)] +
        [f"[g0_{e}] \"v\"(g0[{e}])" for e in range(EPL)] + [f"[q0_{rr}] \"v\"(q0[{rr}])" for rr in range(RB)])
    clob = ", ".join([f"\"v{v}\"" for v in range(lo, 256)] +
                     [f"\"s{s}\"" for s in range(S, SREG_HI + 1)] + ["\"vcc\"", "\"memory\""])
    src = f"""
// Row loop of one wave of the column-split backward, {dtype}, M = {M}, grad_query {DQ}, grad_key {DK}
// (JC = {JC} columns per lane half, {EPL} staged elements per lane, {nmine} private VGPRs).
__device__ __forceinline__ void {name}(float (&dk)[{2*JC}], float (&cs)[{EPL}], const void* g, const void* q,
    void* dq, unsigned qstride, int nfull, int tail, const void* gtail, const void* qtail, unsigned rda,
    unsigned vq, unsigned goff, unsigned gofft, unsigned rs, float vx, float vrt, unsigned kka,
    const unsigned (&st)[{EPL}], unsigned wpar, const unsigned (&g0)[{EPL}], const unsigned (&q0)[{RB}]) {{
  asm volatile(
{asm}
      : {outs}
      : {ins}
      : {clob});
}}
"""
    return name, src, dict(JC=JC, EPL=EPL, HP=HP, PITCH=PITCH, nmine=nmine, RB=RB, XV=XV)


VARIANTS = [(dt, M, dq, dk) for dt in ("f16", "bf16") for M in (49, 32, 16)
            for (dq, dk) in ((True, True), (True, False), (False, True))]


def main(out_path):
    parts = ["// Generated by gen_l1_asm.py from the register map and schedule described there.",
             "// Do not edit by hand: edit the generator and rebuild.", "#pragma once", "namespace lfamd {"]
    for dt, M, dq, dk in VARIANTS:
        name, src, info = variant(dt, M, dq, dk)
        parts.append(f"// {name}: {info}")
        parts.append(src)
    parts.append("}  // namespace lfamd")
    text = "\n".join(parts) + "\n"
    try:
        with open(out_path) as f:
            if f.read() == text:
                return
    except OSError:
        pass
    with open(out_path, "w") as f:
        f.write(text)


if __name__ == "__main__":
    main(sys.argv[1])
