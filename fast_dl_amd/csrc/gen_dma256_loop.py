"""Writes dma256_loop.inc: the steady-state K loop of the four-wave 256x256x16
direct-to-LDS tile (sgemm.hip, CfgDma256W4), as one inline-asm statement.

    python fast_dl_amd/csrc/gen_dma256_loop.py fast_dl_amd/csrc/dma256_loop.inc

The loop is the compiler-scheduled XPIPE loop of sgemm_dma_kernel with three
LDS stages, NN layout, written out instruction by instruction so that every
MFMA, fragment read, copy and wait sits where it is placed here:

  * four waves, one per SIMD, each owning a 128x128 block of the tile: 16
    accumulators of 32x32 (AGPRs, operands %[c00] .. %[c33]);
  * a K-tile is two k-groups of 8; each group is 64 v_mfma_f32_32x32x2_f32 in
    the order (q, mi, ni), so an accumulator is reused every 16 MFMAs;
  * during group 0 the wave reads group 1's fragments of the same tile (slot
    1) and copies A's share of tile t+2; then it waits for tile t+1 (vmcnt 4:
    only those A copies may still be in flight) and its reads, and meets the
    other waves at s_barrier; during group 1 it reads group 0 of tile t+1
    (slot 0) and copies B's share of tile t+2;
  * copies are buffer_load_dwordx4 ... lds: the operand's base in a buffer
    descriptor, a 32-bit lane offset per copy, the K-tile's offset in one
    scalar register advanced once per tile (no per-copy address arithmetic);
  * the stages rotate with the K-tile, so the loop body is three K-tiles long
    and every LDS offset is an immediate.

Fragments live in fixed registers (v160..v223, clobbered by the statement):
slot s, A block mi: v[160 + 32s + 4mi .. +3] (one ds_read_b128: the four k
values of a lane's row in the group); B block ni: v[176 + 32s + 4ni .. +3]
(two ds_read2st64_b32: k rows 1 KB apart).  Reads and copies are spread one
per few MFMAs (a read every 5 MFMAs from the second; the four copies of a
group right after its first four MFMAs), measured on MI355X at 4096^3:
945 us for the compiler-scheduled eight-wave tile, 930 us for this loop with
global_load_lds copies, 915-920 us with buffer copies.
"""
import sys

READ_SLOTS = [1, 6, 11, 16, 21, 26, 31, 36, 41, 46, 51, 56]   # MFMA after which each read goes
COPY_SLOTS = [1, 2, 3, 4]                                     # and each copy
STAGE = 16384                                                 # bytes of one operand's stage


def areg(s, mi):
    return 160 + 32 * s + 4 * mi


def breg(s, ni):
    return 176 + 32 * s + 4 * ni


def reads(slot, g, stage):
    """The 12 fragment reads of k-group g from `stage` into `slot`."""
    out = []
    for mi in range(4):
        r = areg(slot, mi)
        # %[ra<g>]: the lane's row start plus its rotated 16-byte k-chunk
        out.append(f"ds_read_b128 v[{r}:{r + 3}], %[ra{g}] offset:{stage * STAGE + mi * 2048}")
    for ni in range(4):
        r = breg(slot, ni)
        for p in range(2):
            # %[rb<ni>]: the lane's column and k half; offsets in 256-byte units
            o0 = stage * 64 + (8 * g + 2 * p) * 4
            out.append(f"ds_read2st64_b32 v[{r + 2 * p}:{r + 2 * p + 1}], %[rb{ni}] "
                       f"offset0:{o0} offset1:{o0 + 4}")
    return out


def copies(op, stage):
    """Operand op's four copies of a tile into `stage`, and the instruction
    that then advances the operand's K offset to the next tile."""
    out = []
    for i in range(4):
        out.append([f"s_add_u32 m0, %[m{op}{i}], {stage * STAGE}",
                    "s_nop 0",  # M0 written by SALU, then read by an LDS DMA: one wait state
                    f"buffer_load_dwordx4 %[v{op}{i}], %[rs{op}], %[so{op}] offen lds"])
    step = "64" if op == "a" else "%[bstep]"
    return out, f"s_add_u32 %[so{op}], %[so{op}], {step}"


def group(slot, rd, cp):
    out = []
    rd = list(rd)
    cp, advance = cp
    for j in range(64):
        q, mi, ni = j // 16, (j // 4) % 4, j % 4
        out.append(f"v_mfma_f32_32x32x2_f32 %[c{mi}{ni}], v{areg(slot, mi) + q}, "
                   f"v{breg(slot, ni) + q}, %[c{mi}{ni}]")
        if j in READ_SLOTS:
            out.append(rd.pop(0))
        if j in COPY_SLOTS:
            out += cp[COPY_SLOTS.index(j)]
        if j == COPY_SLOTS[-1] + 2:  # two MFMAs after the last copy that reads the offset
            out.append(advance)
    assert not rd
    return out


def ktile(phase):
    cur, nxt, dst = phase, (phase + 1) % 3, (phase + 2) % 3   # stages of tiles t, t+1, t+2
    out = ["s_waitcnt lgkmcnt(0)"]                            # slot 0: group 0 of tile t
    out += group(0, reads(1, 1, cur), copies("a", dst))
    out += ["s_waitcnt vmcnt(4) lgkmcnt(0)", "s_barrier"]     # tile t+1 landed, slot 1 read
    out += group(1, reads(0, 0, nxt), copies("b", dst))
    return out


def main(path):
    lines = ["s_mov_b32 %[m0s], m0",   # M0 is the compiler's: saved and restored
             "s_waitcnt lgkmcnt(0)",
             "s_nop 4"]                # accumulators written just before by VALU
    lines += reads(0, 0, 0)            # group 0 of tile 0
    lines.append("L_fdl_dma256w4_%=:")
    for phase in range(3):
        lines += ktile(phase)
    lines += ["s_sub_u32 %[cnt], %[cnt], 1",
              "s_cmp_lg_u32 %[cnt], 0",
              "s_cbranch_scc1 L_fdl_dma256w4_%=",
              "s_waitcnt lgkmcnt(0)",  # no read may land after the statement
              "s_nop 7", "s_nop 7", "s_nop 7",  # last MFMAs retire before the compiler reads AGPRs
              "s_mov_b32 m0, %[m0s]"]
    out = ["// Generated by gen_dma256_loop.py (same directory); edit that, not this.",
           "// The steady-state K loop of the four-wave 256x256x16 tile (CfgDma256W4).",
           "#pragma once",
           "#define FDL_DMA256W4_LOOP \\"]
    out += [f'    "{line}\\n\\t" \\' for line in lines]
    out.append('    ""')
    with open(path, "w") as f:
        f.write("\n".join(out) + "\n")


if __name__ == "__main__":
    main(sys.argv[1])
