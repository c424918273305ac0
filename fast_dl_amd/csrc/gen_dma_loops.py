"""Writes dma_loops.inc: the hand-scheduled steady-state K loops of the
four-wave direct-to-LDS tiles of sgemm.hip, one inline-asm statement each.

    python fast_dl_amd/csrc/gen_dma_loops.py fast_dl_amd/csrc/dma_loops.inc

Each loop is the compiler-scheduled XPIPE loop of sgemm_dma_kernel with three
LDS stages, for one operand layout (NN, NT, TN or TT), written out
instruction by instruction so that every MFMA, fragment read, copy and wait
sits where it is placed here:

  * four waves, one per SIMD, each owning a WM x WN block of the tile as
    FM x FN accumulators of 32x32 (AGPRs, operands %[c<mi><ni>]);
  * a K-tile is NG k-groups of 8; each group is 4*FM*FN
    v_mfma_f32_32x32x2_f32 in the order (q, mi, ni), so an accumulator is
    reused every FM*FN MFMAs;
  * during group g the wave reads group g+1's fragments (the last group reads
    group 0 of tile t+1) into the other register slot and issues chunk g of
    tile t+2's copies (A's copies first, then B's, spread over the groups as
    sgemm_dma_kernel's three-stage form does); the barrier sits before the
    last group, after a wait for tile t+1 (vmcnt: only tile t+2's chunks
    issued so far may still be in flight) and for the reads;
  * copies are buffer_load_dwordx4 ... lds: the operand's base in a buffer
    descriptor, a 32-bit lane offset per copy, the K-tile's offset in one
    scalar register advanced once per tile (no per-copy address arithmetic);
  * the stages rotate with the K-tile, so the loop body is three K-tiles long
    and every LDS offset is an immediate.

Fragments live in fixed registers from v160 (clobbered by the statement):
slot s, A block mi and B block ni: 4 registers each, the four k values of the
lane's row or column in the group.  A k-contiguous operand (A in NN/NT, B in
NT/TT) is read with one ds_read_b128 from its rotated 16-byte k-chunk; an
mn-contiguous one (A in TN/TT, B in NN/TN) with two ds_read2st64_b32 of k rows
MN floats apart.

For each loop the file defines <NAME>_TEXT (the statement), <NAME>_ACC (its
accumulator operands, acc[mi][ni]) and <NAME>_READS (its fragment read
bases: rka[g][mi] / rkb[g][ni] for a k-contiguous operand, the block's base
for group g; rma[mi] / rmb[ni] for an mn-contiguous one, the lane's column at
k row 4 * half).  Measured on MI355X at 4096^3 (256x256 tile): 945 us
for the compiler-scheduled eight-wave tile, 930 us for this loop with
global_load_lds copies, 911-920 us with buffer copies.
"""
import sys
from dataclasses import dataclass


@dataclass
class Loop:
    macro: str
    bm: int
    bn: int
    bk: int
    wm: int
    wn: int
    read_every: int       # MFMAs between two fragment reads
    copy_slots: tuple     # MFMAs of a group after which its copies go
    a_kc: bool = True     # A k-contiguous (not transposed)
    b_kc: bool = False    # B k-contiguous (transposed)
    ahead: int = 1        # groups between a group's fragment reads and its MFMAs
    nt: int = 256
    stages: int = 3

    @property
    def fm(self):
        return self.wm // 32

    @property
    def fn(self):
        return self.wn // 32

    @property
    def ng(self):
        return self.bk // 8

    @property
    def stage_a(self):
        return self.bm * self.bk * 4

    @property
    def stage_b(self):
        return self.bk * self.bn * 4

    @property
    def per_a(self):
        return self.bm * self.bk // 4 // self.nt

    @property
    def per_b(self):
        return self.bk * self.bn // 4 // self.nt

    def base_per_block(self, blocks):
        """Whether a lane's rotated k-chunk differs between its blocks of a
        k-contiguous operand (the rotation of row r is kc_swz(r); blocks are
        32 rows apart)."""
        cpr = self.bk // 4
        swz = {4: lambda r: (r >> 2) & 3, 8: lambda r: (r ^ (r >> 3)) & 7, 16: lambda r: r & 15}[cpr]
        return any(swz(r) != swz(r + 32 * b) for r in range(64) for b in range(blocks))


def emit(L: Loop) -> list:
    fm, fn, ng, D = L.fm, L.fn, L.ng, L.ahead
    slot_regs = 4 * (fm + fn)
    assert 160 + (D + 1) * slot_regs <= 256 and ng > D and (3 * ng) % (D + 1) == 0
    per_tile = L.per_a + L.per_b
    operands = {}   # read-base operand name -> C++ expression

    def areg(s, mi):
        return 160 + slot_regs * s + 4 * mi

    def breg(s, ni):
        return 160 + slot_regs * s + 4 * fm + 4 * ni

    def kc_reads(x, reg, blocks, g, stage, stage_bytes):
        # k-contiguous rows of BK floats, 16-byte chunks rotated per row
        out = []
        per_block = L.base_per_block(blocks)
        for b in range(blocks):
            r = reg(b)
            if per_block:   # the lane's row start plus its rotated k-chunk, per block
                name, expr, off = f"r{x}{g}{b}", f"rk{x}[{g}][{b}]", stage * stage_bytes
            else:           # block 0's; the blocks are 32 rows apart
                name, expr, off = f"r{x}{g}", f"rk{x}[{g}][0]", stage * stage_bytes + b * 32 * L.bk * 4
            operands[name] = expr
            assert off < 65536
            out.append(f"ds_read_b128 v[{r}:{r + 3}], %[{name}] offset:{off}")
        return out

    def mn_reads(x, reg, blocks, mn, g, stage, stage_bytes):
        # k rows of MN floats; the lane's column at k row 4 * half
        out = []
        row_units = mn * 4 // 256   # one k row, in ds_read2st64's 256-byte units
        for b in range(blocks):
            r = reg(b)
            name = f"r{x}m{b}"
            operands[name] = f"rm{x}[{b}]"
            for p in range(2):
                o0 = stage * stage_bytes // 256 + (8 * g + 2 * p) * row_units
                assert o0 + row_units <= 255
                out.append(f"ds_read2st64_b32 v[{r + 2 * p}:{r + 2 * p + 1}], %[{name}] "
                           f"offset0:{o0} offset1:{o0 + row_units}")
        return out

    def reads(slot, g, stage):
        if L.a_kc:
            out = kc_reads("a", lambda b: areg(slot, b), fm, g, stage, L.stage_a)
        else:
            out = mn_reads("a", lambda b: areg(slot, b), fm, L.bm, g, stage, L.stage_a)
        if L.b_kc:
            out += kc_reads("b", lambda b: breg(slot, b), fn, g, stage, L.stage_b)
        else:
            out += mn_reads("b", lambda b: breg(slot, b), fn, L.bn, g, stage, L.stage_b)
        return out

    def chunk_lo(g):
        return g * per_tile // ng

    def copy(i, stage):
        op, j = ("a", i) if i < L.per_a else ("b", i - L.per_a)
        base = L.stage_a if op == "a" else L.stage_b
        return [f"s_add_u32 m0, %[m{op}{j}], {stage * base}",
                "s_nop 0",   # M0 written by SALU, then read by an LDS DMA: one wait state
                f"buffer_load_dwordx4 %[v{op}{j}], %[rs{op}], %[so{op}] offen lds"]

    def advance(op):   # %[astep], %[bstep]: one K-tile of the operand, in bytes
        return f"s_add_u32 %[so{op}], %[so{op}], %[{op}step]"

    def group(slot, rd, cps, advances):
        out = []
        rd = list(rd)
        n = 4 * fm * fn
        # a read every read_every MFMAs, closer where the layout has more
        # reads, and several after one MFMA where a group has fewer MFMAs
        every = min(L.read_every, (n - 2) // max(1, len(rd) - 1))
        if every > 0:
            slots = [1 + every * i for i in range(len(rd))]
        else:
            slots = [1 + (i * (n - 1)) // len(rd) for i in range(len(rd))]
        assert slots[-1] < n
        last_copy = max(L.copy_slots[:len(cps)]) if cps else -1
        for j in range(n):
            q, mi, ni = j // (fm * fn), (j // fn) % fm, j % fn
            out.append(f"v_mfma_f32_32x32x2_f32 %[c{mi}{ni}], v{areg(slot, mi) + q}, "
                       f"v{breg(slot, ni) + q}, %[c{mi}{ni}]")
            while rd and slots and slots[0] == j:
                slots.pop(0)
                out.append(rd.pop(0))
            for k, cj in enumerate(L.copy_slots[:len(cps)]):
                if cj == j:
                    out += cps[k]
            if j == last_copy + 2:   # two MFMAs after the last copy that reads the offset
                out += advances
        assert not rd
        return out

    reads_per_group = len(reads(0, 0, 0))
    operands.clear()

    def ktile(phase):
        # Group g's fragments were read D groups earlier into register slot
        # (global group index) % (D + 1); during group g the wave reads group
        # g + D, which is in tile t+1 for the last D groups.  The barrier sits
        # before group ng - D, so those reads follow it; it waits for every
        # read of tile t (lgkmcnt 0) and for tile t+1's copies (vmcnt).
        cur, nxt, dst = phase, (phase + 1) % 3, (phase + 2) % 3   # stages of tiles t, t+1, t+2
        out = []
        for g in range(ng):
            gg = phase * ng + g
            if g == ng - D:
                out += [f"s_waitcnt vmcnt({chunk_lo(ng - D)}) lgkmcnt(0)", "s_barrier"]
            else:   # this group's fragments (reads of the D - 1 later groups may fly)
                out.append(f"s_waitcnt lgkmcnt({min(15, (D - 1) * reads_per_group)})")
            if g + D < ng:
                rd = reads((gg + D) % (D + 1), g + D, cur)
            else:
                rd = reads((gg + D) % (D + 1), g + D - ng, nxt)
            ids = range(chunk_lo(g), chunk_lo(g + 1))
            cps = [copy(i, dst) for i in ids]
            advances = []
            if L.per_a - 1 in ids:
                advances.append(advance("a"))
            if per_tile - 1 in ids:
                advances.append(advance("b"))
            out += group(gg % (D + 1), rd, cps, advances)
        return out

    lines = ["s_mov_b32 %[m0s], m0",   # M0 is the compiler's: saved and restored
             "s_waitcnt lgkmcnt(0)",
             "s_nop 4"]                # accumulators written just before by VALU
    for g in range(D):                 # groups 0 .. D-1 of tile 0
        lines += reads(g, g, 0)
    label = f"L_{L.macro.lower()}_%="
    lines.append(f"{label}:")
    for phase in range(3):
        lines += ktile(phase)
    lines += ["s_sub_u32 %[cnt], %[cnt], 1",
              "s_cmp_lg_u32 %[cnt], 0",
              f"s_cbranch_scc1 {label}",
              "s_waitcnt lgkmcnt(0)",  # no read may land after the statement
              "s_nop 7", "s_nop 7", "s_nop 7",  # last MFMAs retire before the compiler reads AGPRs
              "s_mov_b32 m0, %[m0s]"]
    out = [f"#define {L.macro}_TEXT \\"]
    out += [f'    "{line}\\n\\t" \\' for line in lines]
    out.append('    ""')
    acc = [f'[c{mi}{ni}] "+a"(acc[{mi}][{ni}])' for mi in range(fm) for ni in range(fn)]
    out.append(f"#define {L.macro}_ACC " + ", ".join(acc))
    rd = [f'[{k}] "v"({v})' for k, v in operands.items()]
    out.append(f"#define {L.macro}_READS " + ", ".join(rd))
    return out


LAYOUTS = {"NN": (True, False), "NT": (True, True), "TN": (False, False), "TT": (False, True)}
LOOPS = []
for lay, (a_kc, b_kc) in LAYOUTS.items():
    # 256x256x16, waves of 128x128 (CfgDma256W4): a read every 5 MFMAs from
    # the second, a group's four copies after its first four MFMAs.
    LOOPS.append(Loop(f"FDL_DMA256W4_{lay}", 256, 256, 16, 128, 128, read_every=5,
                      copy_slots=(1, 2, 3, 4), a_kc=a_kc, b_kc=b_kc))
    # 128x128x32, waves of 64x64 (CfgDma128W4): four groups of 16 MFMAs, a
    # read every 2 MFMAs, a group's two copies after its first two MFMAs.
    LOOPS.append(Loop(f"FDL_DMA128W4_{lay}", 128, 128, 32, 64, 64, read_every=2,
                      copy_slots=(1, 2), a_kc=a_kc, b_kc=b_kc))
    # 64x64x64, waves of 32x32 (CfgDma64W4): eight groups of 4 MFMAs on one
    # accumulator (a dependent chain costs 69 cycles per MFMA against 65 for
    # independent ones), so each group's fragments are read two groups ahead;
    # one copy per group, after its first MFMA.
    LOOPS.append(Loop(f"FDL_DMA64W4_{lay}", 64, 64, 64, 32, 32, read_every=1,
                      copy_slots=(0,), a_kc=a_kc, b_kc=b_kc, ahead=2))


def main(path):
    out = ["// Generated by gen_dma_loops.py (same directory); edit that, not this.",
           "// Hand-scheduled steady-state K loops of the four-wave direct-to-LDS tiles.",
           "#pragma once"]
    for L in LOOPS:
        out += [""] + emit(L)
    with open(path, "w") as f:
        f.write("\n".join(out) + "\n")


if __name__ == "__main__":
    main(sys.argv[1])
