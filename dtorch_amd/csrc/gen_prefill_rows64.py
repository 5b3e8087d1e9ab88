"""Generate the tile loop of prefill_rows64_kernel (prefill_rows64.hip) as inline-asm programs.

The loop is written out instruction by instruction because its register plan does not fit the compiler's
allocator: a wave keeps 64 query rows (two 32-row blocks A and B sharing every K and V^T fragment), so it
holds O (128 registers) and Q (64) in accumulation registers and two tiles of scores (128), P (32) and
fragment temporaries in vector registers -- over 400 registers at one wave per SIMD.  Left to hipcc the same
loop spills ~250 registers.

Per 64-key tile t the program runs two phases of 32 MFMAs each, software-pipelined across tiles:
  phase A:  S(t+1) = K(t+1) Q^T  (v_mfma_f32_32x32x16, A and B rows on every K fragment)
            || exponentials, row sums and packing of P(t) chunks 0-1 (from S(t)), and tile t+2 / t+1 loads
  phase B:  O += V(t)^T P(t)     (ds_read_b64_tr_b16 fragments, A and B rows on every V^T fragment)
            || P(t) chunks 2-3, then the row max of S(t+1)
followed by the causal / ragged mask of S(t+1) between the phases and the lazy rescale after phase B.  The
arithmetic is that of prefill_fwd_kernel step for step (same fp32 FMA/exp2/sum order, same chains, same
rescale rule per 32-row block), so the two kernels produce identical bits.

Register map (every name is a pinned operand or a clobber of the asm statement):
  VGPR  S[b][X][kt] v[64b + 32X + 16kt : +15]   scores, double-buffered by tile parity b
        P[X][ks]    v[128 + 16X + 4ks : +3]      P chunks in the element type (B operand of O^T += V^T P^T)
        T[s]        v[160 + 4s : +3], s < 5      K / V^T fragment temporaries (read-ahead 4, rotating)
        180+X row max, 182+X swap temp, 184+X max candidate, 186+X alpha, 188+X max base, 190+X mask limit,
        192 -inf, 193..198 rescale temps
        200..207 K fragment addresses (per ks), 208..211 / 212..215 V^T lo / hi addresses (per dt)
        216.. DMA lane offsets (K then V, INSTR each), then the mask lane limits of blocks A and B
  AGPR  O[X][dt] a[64X + 16dt : +15], Q[X][ks] a[128 + 32X + 4ks : +3]
  SGPR  s40 tile t, s41 tile j, s42..s45 temps, s[48:51] K resource, s[52:55] V resource, s[56:63] masks
LDS (byte offsets from the kernel's base, which the address operands include): K buffers at 0 / 16384,
V buffers at 32768 / 49152.

Usage: gen_prefill_rows64.py OUT.inc  -- writes DTATTN_ROWS64_PROGRAM_<BF16|F16>_<NW>_<CAUSAL> and
DTATTN_ROWS64_CLOBBERS.
"""
import sys

NT = 5  # fragment temporaries per stream
MX, TM, MC, AL, MB, LIM, NINF, RT = 180, 182, 184, 186, 188, 190, 192, 193
AK, AVL, AVH, DMA = 200, 208, 212, 216
NEG_FLT_MAX = "0xff7fffff"
SLOT_BUDGET = 30  # issue cycles of VALU work placed after each MFMA (a 32x32x16 MFMA takes 32)
COST = {"v_exp_f32": 16, "v_cvt_pk_": 8, "ds_read": 8, "buffer_load": 8}


def S(buf, X, kt):
    return 64 * buf + 32 * X + 16 * kt


def P(X, ks):
    return 128 + 16 * X + 4 * ks


def T(s):
    return 160 + 4 * s


def O(X, dt):
    return 64 * X + 16 * dt


def Q(X, ks):
    return 128 + 32 * X + 4 * ks


def vr(r, n):
    return f"v[{r}:{r + n - 1}]"


def ar(r, n):
    return f"a[{r}:{r + n - 1}]"


def cost(ins):
    for k, v in COST.items():
        if ins.startswith(k):
            return v
    return 1 if ins.startswith("s_") else 4


class Program:
    def __init__(self, f16, nw, causal):
        self.f16, self.nw, self.causal = f16, nw, causal
        self.instr = 16 // nw  # 1 KB DMA instructions per wave per tile and tensor
        self.lb = DMA + 2 * self.instr  # mask lane limits of blocks A, B
        self.mfma = "v_mfma_f32_32x32x16_f16" if f16 else "v_mfma_f32_32x32x16_bf16"
        self.cvt = "v_cvt_pk_f16_f32" if f16 else "v_cvt_pk_bf16_f32"
        self.L = []

    def e(self, *lines):
        self.L.extend(lines)

    # ---- softmax pieces ----------------------------------------------------------------------------
    def chunk(self, buf, X, ks):
        """P chunk ks of block X from S[buf]: 8 scores -> exp2(s*c - m) (fp32 row sum) -> 4 packed words.
        Software-pipelined per element so that every exponential is read at least one instruction later."""
        kt, half = ks // 2, ks % 2
        regs = [S(buf, X, kt) + 8 * half + e for e in range(8)]
        l = f"%[l{'AB'[X]}]"
        fma = [f"v_fma_f32 v{r}, v{r}, %[c], -v{MB + X}" for r in regs]
        ex = [f"v_exp_f32 v{r}, v{r}" for r in regs]
        add = [f"v_add_f32 {l}, {l}, v{r}" for r in regs]
        cvt = [f"{self.cvt} v{P(X, ks) + j}, v{regs[2 * j]}, v{regs[2 * j + 1]}" for j in range(4)]
        out = []
        for st in range(10):
            if st < 8:
                out.append(fma[st])
            if 1 <= st <= 8:
                out.append(ex[st - 1])
            if st >= 2:
                out.append(add[st - 2])
                if (st - 2) % 2 == 1:
                    out.append(cvt[(st - 2) // 2])
        return out

    @staticmethod
    def rowmax(buf, X):
        regs = [S(buf, X, 0) + i for i in range(16)] + [S(buf, X, 1) + i for i in range(16)]
        out = [f"v_max3_f32 v{MX + X}, v{regs[0]}, v{regs[1]}, v{regs[2]}"]
        for i in range(3, 31, 2):
            out.append(f"v_max3_f32 v{MX + X}, v{MX + X}, v{regs[i]}, v{regs[i + 1]}")
        out.append(f"v_max_f32 v{MX + X}, v{MX + X}, v{regs[31]}")
        # the other half of the wave holds the same rows' other keys
        out += [f"v_mov_b32 v{TM + X}, v{MX + X}", "s_nop 1", f"v_permlane32_swap_b32 v{MX + X}, v{TM + X}",
                f"v_max_f32 v{MX + X}, v{MX + X}, v{TM + X}"]
        return out

    @staticmethod
    def slots(valu, deadlines=()):
        """Place the VALU work after the 32 MFMAs of a phase, at most SLOT_BUDGET issue cycles per slot
        (raised until everything fits and every (slot, count) deadline holds)."""
        b = SLOT_BUDGET
        while True:
            out, i = [], 0
            for _ in range(32):
                sl, c = [], 0
                while i < len(valu) and (not sl or c + cost(valu[i]) <= b):
                    c += cost(valu[i])
                    sl.append(valu[i])
                    i += 1
                out.append(sl)
            ok = i == len(valu)
            cum = 0
            for k in range(32):
                cum += len(out[k])
                ok = ok and all(cum >= cnt for slot, cnt in deadlines if slot == k)
            if ok:
                return out
            b += 2

    # ---- phases ----------------------------------------------------------------------------------------
    def kread(self, kb, f):
        ks, kt = f // 2, f % 2
        return f"ds_read_b128 {vr(T(f % NT), 4)}, v{AK + ks} offset:{kb * 16384 + kt * 8192}"

    def vread(self, vb, g):
        ks, dt = g // 4, g % 4
        off = 32768 + vb * 16384 + ks * 4096
        s = (g + 1) % NT  # clear of K fragment 15's temporary, which the last two MFMAs of phase A read
        return [f"ds_read_b64_tr_b16 {vr(T(s), 2)}, v{AVL + dt} offset:{off}",
                f"ds_read_b64_tr_b16 {vr(T(s) + 2, 2)}, v{AVH + dt} offset:{off}"]

    def phase_a(self, sc, sn, kb, chunks, dma=None, vpre=None):
        """S[sn] = K(buffer kb) Q^T, with the VALU of P chunks from S[sc], DMA pairs by slot and, in the last
        two slots, the first V^T fragment reads of phase B (buffer vpre)."""
        valu = [x for X, ks in chunks for x in self.chunk(sc, X, ks)]
        sl = self.slots(valu)
        self.e("s_waitcnt lgkmcnt(0)", *[self.kread(kb, f) for f in range(4)])
        for m in range(32):
            f = m // 2
            ks, kt, X = f // 2, f % 2, m % 2
            if m % 2 == 0:
                self.e(f"s_waitcnt lgkmcnt({min(3, 15 - f)})")
            d = vr(S(sn, X, kt), 16)
            self.e(f"{self.mfma} {d}, {vr(T(f % NT), 4)}, {ar(Q(X, ks), 4)}, {'0' if ks == 0 else d}")
            if m % 2 == 1 and f + 4 < 16:
                self.e(self.kread(kb, f + 4))
            if dma and m in dma:
                self.e(*dma[m])
            if vpre is not None and m >= 30:
                for g in (2 * (m - 30), 2 * (m - 30) + 1):
                    self.e(*self.vread(vpre, g))
            self.e(*sl[m])

    def phase_b(self, sc, sn, vb, chunks, with_max, pre, skip=()):
        """O += V(buffer vb)^T P, with the VALU of P chunks from S[sc] and (with_max) the row max of S[sn].
        The MFMAs of the P chunks in `skip` (all of whose scores are masked, so P = 0) are left out."""
        valu, done = [], {}
        for X, ks in chunks:
            valu += self.chunk(sc, X, ks)
            done[(X, ks)] = len(valu)
        if with_max:
            valu += self.rowmax(sn, 0) + self.rowmax(sn, 1)
        # P chunk (X, ks) is read by MFMA 8ks + X: complete it three slots earlier (two MFMAs in between)
        sl = self.slots(valu, [(8 * ks + X - 3, n) for (X, ks), n in done.items()])
        if not pre:
            self.e("s_waitcnt lgkmcnt(0)", *[x for g in range(4) for x in self.vread(vb, g)])
        for m in range(32):
            g = m // 2
            ks, dt, X = g // 4, g % 4, m % 2
            if m % 2 == 0:
                self.e(f"s_waitcnt lgkmcnt({2 * min(3, 15 - g)})")
            o = ar(O(X, dt), 16)
            if (X, ks) not in skip:
                self.e(f"{self.mfma} {o}, {vr(T((g + 1) % NT), 4)}, {vr(P(X, ks), 4)}, {o}")
            if m % 2 == 1 and g + 4 < 16:
                self.e(*self.vread(vb, g + 4))
            self.e(*sl[m])

    # ---- mask, rescale ---------------------------------------------------------------------------------
    def mask(self, buf, jreg, lbl):
        """Scores of tile j (SGPR jreg) past Sk or, causal, past each row's diagonal -> -inf."""
        self.e(f"s_lshl_b32 s42, {jreg}, 6", "s_add_i32 s43, s42, 64", "s_cmp_gt_i32 s43, %[sk]",
               f"s_cbranch_scc1 {lbl}_do")
        if self.causal:
            self.e("s_add_i32 s43, s42, 63", "s_cmp_gt_i32 s43, %[kd]", f"s_cbranch_scc1 {lbl}_do")
        # the scores were written by MFMAs: their results need 18 wait states before a VALU read
        self.e(f"s_branch {lbl}_done", f"{lbl}_do:", "s_nop 7", "s_nop 7", "s_nop 4")
        for X in range(2):
            self.e(f"v_subrev_u32 v{LIM + X}, s42, v{self.lb + X}")
        offs = [(kt, i, kt * 32 + 8 * (i >> 2) + (i & 3)) for kt in range(2) for i in range(16)]
        for X in range(2):
            for b0 in range(0, 32, 4):
                batch = offs[b0:b0 + 4]
                self.e(*[f"v_cmp_lt_i32_e64 s[{56 + 2 * n}:{57 + 2 * n}], v{LIM + X}, {off}"
                         for n, (kt, i, off) in enumerate(batch)])
                self.e(*[f"v_cndmask_b32_e64 v{S(buf, X, kt) + i}, v{S(buf, X, kt) + i}, v{NINF}, "
                         f"s[{56 + 2 * n}:{57 + 2 * n}]" for n, (kt, i, off) in enumerate(batch)])
        self.e(f"{lbl}_done:")

    def rescale(self, X, lbl):
        """Lazy rescale of block X: only when some row's max grew by more than 2^8 (wave-uniform)."""
        xn = "AB"[X]
        m, l = f"%[m{xn}]", f"%[l{xn}]"
        self.e(f"v_mul_f32 v{AL + X}, %[c], v{MX + X}",
               f"v_max_f32 v{MC + X}, {m}, v{AL + X}",
               f"v_sub_f32 v{AL + X}, v{MC + X}, {m}",
               f"v_cmp_lt_f32 vcc, 0x41000000, v{AL + X}",
               "s_cmp_eq_u64 vcc, 0",
               f"s_cbranch_scc1 {lbl}_keep",
               f"v_max_f32 v{AL + X}, {NEG_FLT_MAX}, v{MC + X}",  # alpha = exp2(m - mcand), mcand = -inf -> 0
               f"v_sub_f32 v{AL + X}, {m}, v{AL + X}",
               f"v_exp_f32 v{AL + X}, v{AL + X}",
               f"v_cmp_eq_f32 vcc, 0xff800000, {m}",
               "s_cmp_eq_u64 vcc, exec",
               f"s_cbranch_scc1 {lbl}_set",  # every row still at -inf: O and l are exactly 0
               "s_nop 7", "s_nop 7", "s_nop 4",
               f"v_mul_f32 {l}, {l}, v{AL + X}")
        regs = [O(X, dt) + i for dt in range(4) for i in range(16)]
        for b0 in range(0, 64, 6):
            batch = regs[b0:b0 + 6]
            self.e(*[f"v_accvgpr_read_b32 v{RT + n}, a{a}" for n, a in enumerate(batch)])
            self.e(*[f"v_mul_f32 v{RT + n}, v{RT + n}, v{AL + X}" for n, a in enumerate(batch)])
            self.e(*[f"v_accvgpr_write_b32 a{a}, v{RT + n}" for n, a in enumerate(batch)])
        self.e(f"{lbl}_set:", f"v_mov_b32 {m}, v{MC + X}", f"{lbl}_keep:")

    # ---- tile loads ------------------------------------------------------------------------------------
    def dma_setup(self, which, jreg):
        """Buffer resource of tile j of K or V: the tile's rows below Sk; none past the last tile, whose
        loads then land zeros without touching memory."""
        pitch, rs = ("%[kp]", 48) if which == "K" else ("%[vp]", 52)
        w = which.lower()
        return [f"s_lshl_b32 s42, {jreg}, 6", f"s_mul_i32 s43, s42, {pitch}",
                f"s_add_u32 s{rs}, %[{w}lo], s43", f"s_addc_u32 s{rs + 1}, %[{w}hi], 0",
                "s_sub_i32 s44, %[sk], s42", "s_min_i32 s44, s44, 64", "s_add_i32 s44, s44, -1",
                f"s_mul_i32 s{rs + 2}, s44, {pitch}", f"s_add_i32 s{rs + 2}, s{rs + 2}, 256",
                f"s_cmp_lt_i32 {jreg}, %[nt]", f"s_cselect_b32 s{rs + 2}, s{rs + 2}, 0",
                f"s_mov_b32 s{rs + 3}, 0x20000"]

    def dma_pairs(self, which, buf):
        rs = 48 if which == "K" else 52
        lds = (0 if which == "K" else 32768) + buf * 16384
        first = DMA + (0 if which == "K" else self.instr)
        return [[f"s_add_u32 m0, %[m0base], {lds + i * 1024}",
                 f"buffer_load_dwordx4 v{first + i}, s[{rs}:{rs + 3}], 0 offen lds"] for i in range(self.instr)]

    # ---- the loop ----------------------------------------------------------------------------------------
    def tile(self, par, u):
        """Tile t (s40) of parity par: S(t) in S[par]; S(t+1) -> S[1-par] from K buffer 1-par; V(t) in V
        buffer par.  Loads K(t+2) -> K buffer par and V(t+1) -> V buffer 1-par."""
        lb = f"L{u}_%="
        self.e("s_waitcnt vmcnt(0) lgkmcnt(0)", "s_barrier")  # this wave's loads landed; all waves past t-1
        self.e("s_add_i32 s41, s40, 2", *self.dma_setup("K", "s41"))
        self.e("s_add_i32 s41, s40, 1", *self.dma_setup("V", "s41"))
        pairs = self.dma_pairs("K", par) + self.dma_pairs("V", 1 - par)
        flat = [x for p in pairs for x in p]
        self.e("s_cmp_lt_i32 s40, %[tw]", f"s_cbranch_scc1 {lb}_go", *flat, f"s_branch {lb}_next", f"{lb}_go:")
        # max base of the exponentials: m where finite; where m = -inf every score of the row is -inf too
        self.e(f"v_max_f32 v{MB}, {NEG_FLT_MAX}, %[mA]", f"v_max_f32 v{MB + 1}, {NEG_FLT_MAX}, %[mB]")
        self.e("s_add_i32 s41, s40, 1", "s_cmp_lt_i32 s41, %[tw]", f"s_cbranch_scc0 {lb}_last")
        ca = [(0, 0), (1, 0), (0, 1), (1, 1)]
        cb = [(0, 2), (1, 2), (0, 3), (1, 3)]
        step = 32 // len(pairs)
        self.phase_a(par, 1 - par, 1 - par, ca, dma={k * step: pairs[k] for k in range(len(pairs))}, vpre=par)
        self.mask(1 - par, "s41", f"{lb}_m")
        self.phase_b(par, 1 - par, par, cb, True, True)
        self.rescale(0, f"{lb}_ra")
        self.rescale(1, f"{lb}_rb")
        self.e(f"s_branch {lb}_next", f"{lb}_last:", *flat)
        # the wave's last tile: P(t) and O += V(t)^T P(t) only
        if self.causal:
            # On a causal diagonal, block A may see none of the tile's upper 32 keys (every lane's limit
            # below offset 32): its P chunks 2-3 are then exp2(-inf) = 0, adding +0 to the row sums and
            # nothing to O, so their VALU and MFMAs are skipped.
            self.e("s_lshl_b32 s42, s40, 6", f"v_subrev_u32 v{RT}, s42, v{self.lb}",
                   f"v_cmp_gt_i32 vcc, 32, v{RT}", "s_cmp_eq_u64 vcc, exec", f"s_cbranch_scc1 {lb}_diag")
        self.e(*[x for X, ks in ca for x in self.chunk(par, X, ks)])
        self.phase_b(par, 1 - par, par, cb, False, False)
        if self.causal:
            self.e(f"s_branch {lb}_next", f"{lb}_diag:")
            self.e(*[x for X, ks in ca for x in self.chunk(par, X, ks)])
            self.phase_b(par, 1 - par, par, cb[1:2] + cb[3:], False, False, skip=((0, 2), (0, 3)))
        self.e(f"{lb}_next:", "s_add_i32 s40, s40, 1")

    def program(self):
        self.e(f"v_mov_b32 v{NINF}, 0xff800000")
        # S(0) -> S[0] from K buffer 0, its mask, row max and the first max update
        self.e("s_cmp_gt_i32 %[tw], 0", "s_cbranch_scc0 L_p_%=_end")
        self.phase_a(1, 0, 0, [])
        self.e("s_mov_b32 s41, 0")
        self.mask(0, "s41", "L_p_%=_m")
        self.e("s_nop 7", "s_nop 7", "s_nop 4", *self.rowmax(0, 0), *self.rowmax(0, 1))
        self.rescale(0, "L_p_%=_ra")
        self.rescale(1, "L_p_%=_rb")
        self.e("L_p_%=_end:", "s_mov_b32 s40, 0", "L_top_%=:")
        self.tile(0, "e")
        self.e("s_cmp_lt_i32 s40, %[nt]", "s_cbranch_scc0 L_end_%=")
        self.tile(1, "o")
        # the loads past the last tile may still be in flight: land them before the LDS is reused; the last
        # MFMAs' results need their wait states before the compiler's code reads O
        self.e("s_cmp_lt_i32 s40, %[nt]", "s_cbranch_scc1 L_top_%=", "L_end_%=:", "s_waitcnt vmcnt(0)",
               "s_nop 7", "s_nop 7", "s_nop 4")
        return self.L


def main(path):
    out = ["// Generated by gen_prefill_rows64.py: do not edit.\n#pragma once\n"]
    for f16 in (False, True):
        for nw in (2, 4):
            for causal in (False, True):
                lines = Program(f16, nw, causal).program()
                out.append(f"#define DTATTN_ROWS64_PROGRAM_{'F16' if f16 else 'BF16'}_{nw}_{int(causal)} \\")
                out.append(" \\\n".join('    "' + l + '\\n"' for l in lines))
                out.append("")
    clob = ", ".join(f'"v{i}"' for i in range(200)) + ", " + ", ".join(f'"s{i}"' for i in range(40, 64))
    out.append(f'#define DTATTN_ROWS64_CLOBBERS {clob}, "vcc", "m0", "memory"')
    tmp = path + ".tmp"
    with open(tmp, "w") as fh:
        fh.write("\n".join(out) + "\n")
    import os
    os.replace(tmp, path)


if __name__ == "__main__":
    main(sys.argv[1])
