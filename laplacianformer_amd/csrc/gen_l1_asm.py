#!/usr/bin/env python3
"""Generator of the hand-scheduled gfx950 inner loops of the L1 kernels.

Writes ``l1_asm_gen.h``: ``__device__`` functions each holding a single
``asm volatile`` block:

* ``bwd2_rows_*``: the row loop of one wave of the column-split backward
  (``laplace_bwd2.hip``), per element type, key count M and grad_query /
  grad_key selection. The grad rows are already staged in LDS by the
  workgroup (2g as fp32, each half row 16-byte aligned, the half's sum of g in
  slot JC); the block reads them back, loads the query row of each step, and
  issues the arithmetic and the grad_query stores.
* ``fwd2_sums_*``: the channel loop of the row-staged forward
  (``laplace_fwd2.hip``) for R row sets per lane.

They are generated rather than written by hand because their value lies in
the schedule and the register map:

* every VALU instruction reads VGPR operands only (an SGPR in src1, which
  needs the VOP3 encoding, lowers the issue rate on gfx950);
* ``v_fmac_f32``'s src0 is never in the accumulator's VGPR bank (register
  number mod 4): each product has two candidate src0 registers, the grad value
  and the step value, in different banks, and the generator picks the one that
  differs;
* LDS and global waits are exact counts of the operations issued since the one
  needed, and dependent work is interleaved with independent work across rows
  (backward) or one channel ahead (forward);
* the loop heads are aligned to 64 bytes (``.p2align 6``): the forward lost
  ~0.1 us when an unrelated change to its kernel moved its loop head;
* nothing needs software wait states (the compiler does not insert them
  inside inline asm): there are no DPP, permlane or VALU-written SGPR reads;
* every block names what it writes besides its operands in its clobber list,
  SCC included (its loop control compares and branches on it).

The backward arithmetic per (row i, key column j, channel c), with T() the
order-preserving map of a 16-bit float pattern onto the fp32 values
2^22 + 2^14 + t/2 (t = signed magnitude of the pattern, so +0 and -0 coincide):

    y   = clamp(T(q[i,c]) + (0.5 - T(k[c,j])))      # (sgn(q - k) + 1) / 2, exact
    dq += (2 g[i,j]) * y                            # grad_query: sum_j 2g y - sum_j g
    dk[j] += (2 g[i,j]) * y                         # grad_key:  sum_i g - sum_i 2g y

Run as ``python gen_l1_asm.py <out.h>`` (the build does this).
"""
from __future__ import annotations

import sys

LANES = 64
UNROLL = 4        # rows per loop iteration (= depth of the query prefetch ring)
KK_GSTRIDE = (LANES + 1) * 16   # bytes between 16-byte groups of the key-term table ([group][65][4] floats)
STORE_POLICY = " nt"


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


def shape(M):
    """(JC, HP, NG, PITCH): columns per lane half, LDS slots per half row (JC
    columns, the row sum, padding to 16 bytes), 16-byte groups per half row,
    floats per staged row (both halves and 16 bytes of bank padding)."""
    JC = (M + 1) // 2
    HP = ((JC + 1 + 3) // 4) * 4
    return JC, HP, HP // 4, 2 * HP + 4


def variant(dtype, M, DQ=True, DK=True, top=256):
    """Returns (name, C++ source, info) of the row-loop block for key count M,
    using VGPRs below `top` (256: two waves per SIMD; 168: three).

    With top < 256 the grad_key accumulators and the per-lane inputs are
    operands bound to the block's own registers ("{vN}" constraints) rather
    than copied in and out, so that the compiler holds no second copy of them
    around the block.

    DQ / DK select the grad_query and grad_key halves of the work: without DK
    there are no grad_key accumulators, without DQ no grad_query accumulation
    or stores (the query rows are still needed for the steps).

    Lane (h, p) holds its two channels in the order (own, partner): c0 =
    2p + h, c1 = 2p + 1 - h, so that the grad_query partial a lane owes its
    partner (lane p + 32 (1 - h), the other column half) is always the c1
    accumulator: one ds_bpermute_b32 exchanges them (v_permlane32_swap costs
    the SIMD about ten times a v_fmac).

    Software pipelining across rows: T(q) of row r + 1 is computed during row
    r, and the grad_query of row r is finished during row r + 1 (the partials
    exchanged after its first group, summed, rounded and stored a few groups
    later), so no instruction waits on a just-written operand; the
    accumulators and T(q) alternate between two register sets by row parity.
    Each half subtracts its own half of the row sum (slot JC of the staged
    half row) at the end of the row."""
    assert DQ or DK
    JC, HP, NG, PITCH = shape(M)
    RSLOT = JC
    assert RSLOT // 4 == NG - 1 and NG >= 3
    bf16 = dtype == "bf16"

    phys = top < 256
    r = Regs(top)
    KK = r.take(4 * ((2 * JC + 3) // 4), align=4)   # 0.5 - T(k): [c][j] packed, read as b128 groups
    DK_ = r.take(2 * JC, bank=1) if DK else None      # grad_key accumulators [c][j]
    G = r.take(16, align=4)                           # grad ring: 4 slots of 4 (bank k for element k)
    Y = r.take(8, bank=3)                             # step values [c][k]
    DQA = [[r.take(1, bank=1), r.take(1, bank=2)] for _ in range(2)] if DQ else None  # grad_query [parity][c0, c1]
    RECV = r.take(1) if DQ else None                  # the partner's c1 partial (= this lane's channel)
    TQ = [r.take(2, bank=1) for _ in range(2)]        # T(q) [parity][c]
    QR = r.take(UNROLL)                               # query pattern pairs of the next rows (ring)
    RDA = r.take(1)       # LDS byte address of the current iteration's first row (lane's half)
    VQ4 = r.take(1)       # byte offset of the lane's channel pair in a query row
    VQS = r.take(1)       # byte offset of the lane's own channel in a grad_query row
    T0 = r.take(4)        # T-map temporaries
    FT = r.take(1)        # grad_query finishing temporary
    SHF = r.take(4)       # bit offsets in the query pair: c0 value, c0 sign, c1 value, c1 sign
    PADDR = r.take(1)     # ds_bpermute address of the partner lane
    lo = r.next
    assert lo >= 0
    nmine = top - lo

    # SGPRs (clobbered).
    S = 72
    SQ = S                # 64-bit: query row of the latest prefetch
    SQL = S + 2           # 64-bit: the wave's last query row (prefetch clamp)
    SD = S + 4            # 64-bit: grad_query row of the next store
    SQS = S + 6           # row stride (bytes)
    SLEFT = S + 7         # rows left, counted at iteration starts
    SPR = S + 8           # priority phase
    SPC = S + 9           # iterations until the next priority flip
    STMP = S + 10         # 64-bit temporary (prefetch address)
    SRN = S + 12          # row index of the latest prefetch
    SROWS = S + 13        # rows of the wave
    SDN = S + 14          # 64-bit temporary (next grad_query row)
    SFLAG = S + 16        # 0 until the first (placeholder) grad_query store
    SREG_HI = S + 16

    L = []
    add = L.append

    def grp_cols(g):
        return [j for j in range(4 * g, min(JC, 4 * g + 4))]

    def fmac(acc, gk, yk):
        """v_fmac acc += gk * yk with src0 in a bank different from acc's."""
        if gk % 4 != acc % 4:
            return f"v_fmac_f32 v{acc}, v{gk}, v{yk}"
        return f"v_fmac_f32 v{acc}, v{yk}, v{gk}"

    def tmap(x, tq):
        # T of the lane's c0 and c1 patterns (bit offsets per lane): as_float(0x4a808000 + t),
        # t = +-magnitude.
        for c in range(2):
            add(f"v_bfe_u32 v{T0}, v{x}, v{SHF + 2*c}, 15")
            add(f"v_bfe_i32 v{T0 + 1}, v{x}, v{SHF + 2*c + 1}, 1")
            add(f"v_sub_u32 v{T0 + 2}, 0x4a808000, v{T0 + 1}")
            add(f"v_xad_u32 v{tq + c}, v{T0}, v{T0 + 1}, v{T0 + 2}")

    def finish_store(pp):
        # The lane's own channel: its c0 partial (its column half) plus the
        # partner's c1 partial (the other half), received by ds_bpermute. The
        # very first store of the wave is a placeholder at the first row,
        # rewritten by that row's own store.
        add(f"v_add_f32 v{FT}, v{DQA[pp][0]}, v{RECV}")
        if bf16:
            add(f"v_cvt_pk_bf16_f32 v{FT}, v{FT}, v{FT}")
        else:
            add(f"v_cvt_f16_f32 v{FT}, v{FT}")
        add(f"global_store_short v{VQS}, v{FT}, s[{SD}:{SD+1}]" + STORE_POLICY)
        add(f"s_add_u32 s{SDN}, s{SD}, s{SQS}")
        add(f"s_addc_u32 s{SDN+1}, s{SD+1}, 0")
        add(f"s_cmp_lg_u32 s{SFLAG}, 0")
        add(f"s_cselect_b64 s[{SD}:{SD+1}], s[{SDN}:{SDN+1}], s[{SD}:{SD+1}]")
        add(f"s_mov_b32 s{SFLAG}, 1")

    # ---- entry ---------------------------------------------------------------
    add("s_waitcnt vmcnt(0) lgkmcnt(0)")
    add(f"s_mov_b64 s[{SQ}:{SQ+1}], %[q3]")
    add(f"s_mov_b64 s[{SQL}:{SQL+1}], %[ql]")
    add(f"s_mov_b64 s[{SD}:{SD+1}], %[dq]")
    add(f"s_mov_b32 s{SQS}, %[qs]")
    add(f"s_mov_b32 s{SLEFT}, %[rows]")
    add(f"s_mov_b32 s{SROWS}, %[rows]")
    add(f"s_mov_b32 s{SRN}, {UNROLL - 1}")
    add(f"s_mov_b32 s{SPR}, %[wpar]")
    add(f"s_mov_b32 s{SPC}, 0")
    add(f"s_mov_b32 s{SFLAG}, 0")
    if not phys:
        add(f"v_mov_b32 v{RDA}, %[rda]")
        add(f"v_mov_b32 v{VQ4}, %[vq4]")
        add(f"v_mov_b32 v{VQS}, %[vqs]")
        for c in range(4):
            add(f"v_mov_b32 v{SHF + c}, %[shf{c}]")
        add(f"v_mov_b32 v{PADDR}, %[paddr]")
        for k in range(UNROLL):
            add(f"v_mov_b32 v{QR + k}, %[q0_{k}]")
    kka = f"v{T0}" if phys else "%[kka]"
    for i in range((2 * JC + 3) // 4):
        add(f"ds_read_b128 v[{KK + 4*i}:{KK + 4*i + 3}], {kka} offset:{i * KK_GSTRIDE}")
    if DK and not phys:
        for j in range(2 * JC):
            add(f"v_mov_b32 v{DK_ + j}, %[dk{j}]")
    tmap(QR, TQ[0])
    add("s_waitcnt lgkmcnt(0)")

    ring = 4
    ahead = 3
    # VMEM operations per row: the prefetch load, then the grad_query store.
    # T(q) of row r + 1 is computed in row r: its load (issued in row r - 3) is
    # followed by that row's store and two operations in each of rows r - 2,
    # r - 1 and r.
    vmc = 7 if DQ else 3
    # Group after which the previous row's grad_query is stored: the exchange
    # (issued after group 0) is older than the group's g_fin reads.
    g_fin = min(ahead, NG - 1)
    g_tmap = NG - 2               # group after which T(q) of the next row is computed

    def pos_addr(p):
        rr, g = divmod(p, NG)
        return (rr * PITCH + 4 * g) * 4

    for p in range(ahead):
        add(f"ds_read_b128 v[{G + 4*(p % ring)}:{G + 4*(p % ring) + 3}], v{RDA} offset:{pos_addr(p)}")

    add(".p2align 6")
    add("RL_%=:")
    # Priority: the waves sharing a SIMD (two, or three with top < 256; wpar =
    # the wave's place among them) take turns at the higher issue priority, 8
    # rows each, so that none runs ahead and finishes alone.
    add(f"s_sub_u32 s{SPC}, s{SPC}, 1")
    add(f"s_cmp_lt_i32 s{SPC}, 0")
    add("s_cbranch_scc0 PR_%=_d")
    add(f"s_mov_b32 s{SPC}, {8 // UNROLL - 1}")
    if phys:
        add(f"s_add_u32 s{SPR}, s{SPR}, 1")
        add(f"s_cmp_ge_u32 s{SPR}, 3")
        add(f"s_cselect_b32 s{SPR}, 0, s{SPR}")
    else:
        add(f"s_xor_b32 s{SPR}, s{SPR}, 1")
    add(f"s_cmp_eq_u32 s{SPR}, 0")
    add("s_cbranch_scc1 PR_%=_lo")
    add("s_setprio 2")
    add("s_branch PR_%=_d")
    add("PR_%=_lo:")
    add("s_setprio 0")
    add("PR_%=_d:")
    for rr in range(UNROLL):
        par = rr % 2
        if rr > 0:
            add(f"s_cmp_le_u32 s{SLEFT}, {rr}")
            add(f"s_cbranch_scc1 RX{rr}_%=")
        x = QR + rr
        # Prefetch the query pair UNROLL rows ahead into this row's slot (its T(q)
        # was taken in the previous row); past the wave's last row the last row is
        # read again (never out of bounds).
        add(f"s_add_u32 s{SQ}, s{SQ}, s{SQS}")
        add(f"s_addc_u32 s{SQ+1}, s{SQ+1}, 0")
        add(f"s_add_u32 s{SRN}, s{SRN}, 1")
        add(f"s_cmp_ge_u32 s{SRN}, s{SROWS}")
        add(f"s_cselect_b64 s[{STMP}:{STMP+1}], s[{SQL}:{SQL+1}], s[{SQ}:{SQ+1}]")
        add(f"global_load_dword v{x}, v{VQ4}, s[{STMP}:{STMP+1}]")
        for g in range(NG):
            p = rr * NG + g
            pn = p + ahead
            add(f"ds_read_b128 v[{G + 4*(pn % ring)}:{G + 4*(pn % ring) + 3}], v{RDA} offset:{pos_addr(pn)}")
            add(f"s_waitcnt lgkmcnt({g_fin if DQ and g == g_fin else ahead})")
            gs = G + 4 * (p % ring)
            cols = grp_cols(g)
            for c in range(2):
                for k, j in enumerate(cols):
                    add(f"v_add_f32_e64 v{Y + 4*c + k}, v{TQ[par] + c}, v{KK + c*JC + j} clamp")
            for k, j in enumerate(cols):
                for c in range(2):
                    if DQ:
                        if j == 0:
                            add(f"v_mul_f32 v{DQA[par][c]}, v{gs + k}, v{Y + 4*c + k}")
                        else:
                            add(fmac(DQA[par][c], gs + k, Y + 4*c + k))
                    if DK:
                        add(fmac(DK_ + c*JC + j, gs + k, Y + 4*c + k))
            if DQ and g == 0:
                add(f"ds_bpermute_b32 v{RECV}, v{PADDR}, v{DQA[1 - par][1]}")
            if DQ and g == g_fin:
                finish_store(1 - par)
            if g == g_tmap:
                # T(q) of the next row, into the other parity's registers.
                add(f"s_waitcnt vmcnt({vmc})")
                tmap(QR + (rr + 1) % UNROLL, TQ[1 - par])
        if DQ:
            # This row's grad_query: minus the lane's half of the row sum.
            rg = G + 4 * ((rr * NG + NG - 1) % ring) + (RSLOT % 4)
            for c in range(2):
                add(f"v_sub_f32 v{DQA[par][c]}, v{DQA[par][c]}, v{rg}")
    add(f"v_add_u32 v{RDA}, {UNROLL * PITCH * 4}, v{RDA}")
    add(f"s_sub_u32 s{SLEFT}, s{SLEFT}, {UNROLL}")
    add(f"s_cmp_gt_i32 s{SLEFT}, 0")
    add("s_cbranch_scc1 RL_%=")
    # Exits: the grad_query of the last computed row is still to be stored.
    for rr in (UNROLL, 1, 2, 3):
        if rr != UNROLL:
            add(f"RX{rr}_%=:")
        if DQ:
            pp = (rr - 1) % 2
            add(f"ds_bpermute_b32 v{RECV}, v{PADDR}, v{DQA[pp][1]}")
            add("s_waitcnt lgkmcnt(0)")
            finish_store(pp)
        add("s_branch RX_%=")
    add("RX_%=:")
    add("s_setprio 0")
    add("s_waitcnt vmcnt(0) lgkmcnt(0)")
    if DK and not phys:
        for j in range(2 * JC):
            add(f"v_mov_b32 %[dk{j}], v{DK_ + j}")

    # ---- C++ wrapper -----------------------------------------------------------
    name = f"bwd2_rows_{dtype}_m{M}_{'q' if DQ else ''}{'k' if DK else ''}" + ("" if top == 256 else f"_v{top}")
    asm = "\n".join("      \"" + s + "\\n\"" for s in L)
    sins = ["[q3] \"s\"(q3)", "[ql] \"s\"(qlast)", "[dq] \"s\"(dq)", "[qs] \"s\"(qstride)", "[rows] \"s\"(rows)",
            "[wpar] \"s\"(wpar)"]
    bound = set()
    if phys:
        # Operands in the block's registers: the accumulators, and the inputs the
        # block consumes in place (declared read-write: their values change).
        outl = [f"[dk{j}] \"+{{v{DK_ + j}}}\"(dk[{j}])" for j in range(2 * JC)] if DK else []
        bound.update(range(DK_, DK_ + 2 * JC) if DK else [])
        pairs = [("rda", RDA), ("vq4", VQ4), ("vqs", VQS), ("kka", T0), ("paddr", PADDR)] + \
                [(f"shf[{c}]", SHF + c) for c in range(4)] + [(f"q0[{k}]", QR + k) for k in range(UNROLL)]
        for var, reg in pairs:
            outl.append(f"[i_{reg}] \"+{{v{reg}}}\"({var})")
            bound.add(reg)
        outs = ", ".join(outl)
        ins = ", ".join(sins)
    else:
        outs = ", ".join([f"[dk{j}] \"+v\"(dk[{j}])" for j in range(2 * JC)]) if DK else ""
        ins = ", ".join(sins + [
            "[rda] \"v\"(rda)", "[vq4] \"v\"(vq4)", "[vqs] \"v\"(vqs)", "[kka] \"v\"(kka)",
            "[paddr] \"v\"(paddr)"] + [f"[shf{c}] \"v\"(shf[{c}])" for c in range(4)] +
            [f"[q0_{k}] \"v\"(q0[{k}])" for k in range(UNROLL)])
    clob = ", ".join([f"\"v{v}\"" for v in range(lo, top) if v not in bound] +
                     [f"\"s{s}\"" for s in range(S, SREG_HI + 1)] + ["\"vcc\"", "\"scc\"", "\"memory\""])
    # The block writes the bound inputs: it gets copies of the arrays.
    copies = ("\n  unsigned shf[4] = {shf_[0], shf_[1], shf_[2], shf_[3]};\n  unsigned q0[" + str(UNROLL) + "] = {" +
              ", ".join(f"q0_[{k}]" for k in range(UNROLL)) + "};") if phys else ""
    src = f"""
// Row loop of one wave of the column-split backward, {dtype}, M = {M}, grad_query {DQ}, grad_key {DK}
// (JC = {JC} columns per lane half, LDS row pitch {PITCH} floats, {nmine} private VGPRs).
// rows >= 1 rows; q0: the query pairs of the first {UNROLL} rows (loaded by the caller,
// rows past the wave's end repeat its last row); q3: the query row {UNROLL - 1} rows after the
// first (prefetches advance from it); qlast: the wave's last query row; dq: the first
// grad_query row; rda: LDS address of the first staged row plus the lane's half offset;
// shf: bit offsets of the lane's c0 value, c0 sign, c1 value, c1 sign in a query pair;
// paddr: 4 * (the partner lane).
__device__ __forceinline__ void {name}(float (&dk)[{2*JC}], const void* q3, const void* qlast, void* dq,
    unsigned qstride, int rows, unsigned wpar, unsigned rda, unsigned vq4, unsigned vqs, unsigned kka,
    unsigned paddr, {"const unsigned (&shf_)[4], const unsigned (&q0_)[" + str(UNROLL) + "]" if phys else "const unsigned (&shf)[4], const unsigned (&q0)[" + str(UNROLL) + "]"}) {{{copies}
  asm volatile(
{asm}
      : {outs}
      : {ins}
      : {clob});
}}
"""
    return name, src, dict(JC=JC, HP=HP, PITCH=PITCH, nmine=nmine)


FWD_JB = 7          # key columns per forward column block
FWD_KP = 56 * 4     # bytes per channel of the forward key tile ([C][56] fp32)


def fwd_variant(R, top=256, jb=FWD_JB, kp=FWD_KP, prefix="fwd2"):
    """Returns (name, C++ source) of the channel loop of the row-staged forward
    (laplace_fwd2.hip) for R row sets per lane, using VGPRs below `top` (256:
    two waves per SIMD; 128: four), for blocks of `jb` key columns (7 for M = 49;
    8 for the wide-landmark kernel) in a key tile of `kp` bytes per channel.

    Per channel c and row set s: T = q[s][c] - k[c][j] (v_sub_f32) and
    acc[s][j] += |T| (v_add_f32 with the |.| modifier), j < 7, channels in
    ascending order. The query tile is read as 16-byte vectors (4 channels of
    one row per lane), one group ahead; the key row of a channel as two
    16-byte reads (7 columns + padding), one channel ahead. Eight channels per
    loop iteration (two query groups, so the two query buffers alternate
    statically). Register banks: K[j] and acc[s][j] in bank j % 4, query
    channel cc in bank cc; each T is placed in a bank different from both its
    source query register (the sub's src0) and its accumulator (the add reads
    T as src0 and writes the accumulator)."""
    r = Regs(top)
    QA = [r.take(4, align=4) for _ in range(R)]
    QB = [r.take(4, align=4) for _ in range(R)]
    KS = [r.take(8, align=4) for _ in range(2)]
    ACC = r.take(8 * R, align=4)            # acc[s][j] = ACC + 8s + j (bank j % 4)
    TB = r.take(16, align=4)                # temporaries: bank b holds TB + b, TB + 4 + b, ...
    QADDR = [r.take(1) for _ in range(R)]
    KADDR = r.take(1)
    lo = r.next
    SC = 72
    L = []
    add = L.append

    def acc(s, j):
        return ACC + 8 * s + j

    add("s_waitcnt vmcnt(0) lgkmcnt(0)")
    add(f"s_mov_b32 s{SC}, %[iters]")
    for s_ in range(R):
        add(f"v_mov_b32 v{QADDR[s_]}, %[qa{s_}]")
    add(f"v_mov_b32 v{KADDR}, %[ka]")
    for s_ in range(R):
        for j in range(jb):
            add(f"v_mov_b32 v{acc(s_, j)}, 0")
    for s_ in range(R):
        add(f"ds_read_b128 v[{QA[s_]}:{QA[s_] + 3}], v{QADDR[s_]}")
    add(f"ds_read_b128 v[{KS[0]}:{KS[0] + 3}], v{KADDR}")
    add(f"ds_read_b128 v[{KS[0] + 4}:{KS[0] + 7}], v{KADDR} offset:16")
    add(".p2align 6")
    add("FL_%=:")
    for ci in range(8):
        Q = QA if ci < 4 else QB
        cc = ci % 4
        K = KS[ci % 2]
        Kn = KS[(ci + 1) % 2]
        nq = 0
        if ci == 0 or ci == 4:
            dst = QB if ci == 0 else QA
            off = 16 if ci == 0 else 32
            for s_ in range(R):
                add(f"ds_read_b128 v[{dst[s_]}:{dst[s_] + 3}], v{QADDR[s_]} offset:{off}")
            nq = R
        koff = (ci + 1) * kp
        add(f"ds_read_b128 v[{Kn}:{Kn + 3}], v{KADDR} offset:{koff}")
        add(f"ds_read_b128 v[{Kn + 4}:{Kn + 7}], v{KADDR} offset:{koff + 16}")
        add(f"s_waitcnt lgkmcnt({nq + 2})")
        for s_ in range(R):
            qreg = Q[s_] + cc
            used = [0, 0, 0, 0]
            ts = []
            for j in range(jb):
                ok = [b for b in range(4) if b != qreg % 4 and b != acc(s_, j) % 4 and used[b] < 4]
                b = min(ok, key=lambda b: used[b])
                t = TB + 4 * used[b] + b
                used[b] += 1
                ts.append(t)
                add(f"v_sub_f32 v{t}, v{qreg}, v{K + j}")
            for j in range(jb):
                add(f"v_add_f32_e64 v{acc(s_, j)}, |v{ts[j]}|, v{acc(s_, j)}")
    for s_ in range(R):
        add(f"v_add_u32 v{QADDR[s_]}, 32, v{QADDR[s_]}")
    add(f"v_add_u32 v{KADDR}, {8 * kp}, v{KADDR}")
    add(f"s_sub_u32 s{SC}, s{SC}, 1")
    add(f"s_cmp_gt_u32 s{SC}, 0")
    add("s_cbranch_scc1 FL_%=")
    add("s_waitcnt lgkmcnt(0)")
    for s_ in range(R):
        for j in range(jb):
            add(f"v_mov_b32 %[a{s_}_{j}], v{acc(s_, j)}")

    name = f"{prefix}_sums_r{R}"
    asm = "\n".join("      \"" + x + "\\n\"" for x in L)
    outs = ", ".join(f"[a{s_}_{j}] \"=v\"(acc[{s_}][{j}])" for s_ in range(R) for j in range(jb))
    ins = ", ".join(["[iters] \"s\"(iters)", "[ka] \"v\"(ka)"] + [f"[qa{s_}] \"v\"(qa[{s_}])" for s_ in range(R)])
    clob = ", ".join([f"\"v{v}\"" for v in range(lo, top)] + [f"\"s{SC}\"", "\"scc\"", "\"memory\""])
    if top != 256:
        name += f"_v{top}"
    src = f"""
// Channel loop of the row-staged forward for {R} row set(s) per lane ({top - lo} private VGPRs below v{top}):
// acc[s][j] = sum over channels c < 8 * iters of |q[s][c] - k[c][j]|, c ascending. qa[s]: LDS
// byte address of the lane's row of set s in the fp32 query tile (channel 0); ka: LDS byte
// address of the lane's 8-column key block at channel 0 (rows of {kp} bytes). Reads go one
// query group and one channel past the end (the tiles' padding and the next tile; unused).
__device__ __forceinline__ void {name}(float (&acc)[{R}][{jb}], const unsigned (&qa)[{R}], unsigned ka, int iters) {{
  asm volatile(
{asm}
      : {outs}
      : {ins}
      : {clob});
}}
"""
    return name, src


FWD_RS = (1, 2, 3, 4, 5, 6, 7)
FWD3_KP = 256 * 4   # bytes per channel of the wide-landmark kernel's key tile ([C][256] fp32)
FWD3_RS = (3,)
FWD_RS_V128 = (1, 2, 3)


VARIANTS = [(dt, M, dq, dk) for dt in ("f16", "bf16") for M in (32, 16)
            for (dq, dk) in ((True, True), (True, False), (False, True))]
# M = 49 runs in 12-wave workgroups (three waves per SIMD, 168 VGPRs).
VARIANTS_V168 = [(dt, 49, dq, dk) for dt in ("f16", "bf16")
                 for (dq, dk) in ((True, True), (True, False), (False, True))]


def main(out_path):
    parts = ["// Generated by gen_l1_asm.py from the register map and schedule described there.",
             "// Do not edit by hand: edit the generator and rebuild.", "#pragma once", "namespace lfamd {"]
    for dt, M, dq, dk in VARIANTS:
        name, src, info = variant(dt, M, dq, dk)
        parts.append(f"// {name}: {info}")
        parts.append(src)
    for dt, M, dq, dk in VARIANTS_V168:
        name, src, info = variant(dt, M, dq, dk, top=168)
        parts.append(f"// {name}: {info}")
        parts.append(src)
    for R in FWD_RS:
        name, src = fwd_variant(R)
        parts.append(f"// {name}")
        parts.append(src)
    for R in FWD_RS_V128:
        name, src = fwd_variant(R, 128)
        parts.append(f"// {name}")
        parts.append(src)
    for R in FWD3_RS:
        name, src = fwd_variant(R, 128, jb=8, kp=FWD3_KP, prefix="fwd3")
        parts.append(f"// {name}")
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
