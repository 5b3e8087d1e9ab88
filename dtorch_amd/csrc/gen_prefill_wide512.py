"""Generate the tile loop of prefill_wide512_kernel (prefill_wide512.hip) as inline-asm programs.

The kernel is the head-dim-512 attention of prefill_wide_kernel (non-causal, unmasked, no padding): a
workgroup of 4 waves owns 64 query rows, as 2 row groups of 32 rows times 2 halves of the head dims; wave
(rg, dh) holds Q and accumulates O for its rows and dims [256 dh, 256 dh + 256), and the two waves of a row
group add their partial scores through LDS.  Written by the compiler, each 32-key tile ran as a chain of
dependent phases (partial scores, exchange, softmax, PV) with no overlap, at one wave per SIMD.  Here one
step of the loop runs, for tile t:

  phase A:  S(t+1) partial = K(t+1) Q^T (16 MFMAs, K fragments read four ahead)
            || the partner's partial of S(t), the row max, the lazy-rescale decision and the first half of
               P(t) (VALU), and the loads of K(t+2) (one per MFMA)
  (rare)    O *= alpha
  phase B:  O^T += V(t)^T P(t)^T (16 MFMAs, V^T fragments read four ahead)
            || the second half of P(t), due before the MFMAs that read it, and the loads of V(t+1); then this
               wave's partial of S(t+1) into the exchange slab of the other parity
  one barrier per step.

The arithmetic is that of prefill_wide_kernel element for element (the same MFMA accumulation order, the
same fp32 FMA / exp2 / sum order, the same rescale rule), so the two kernels return identical bits.

Register map (pinned operands or clobbers of the asm statement):
  VGPR  S[b]      v[16b : 16b+15]   this wave's partial scores of the tile of parity b (then the tile's scores,
                                     then its exponentials in place)
        PT        v[32:47]          the partner's partial
        P[h]      v[48 + 4h : +3]   P in the element type, keys of PV k-step h
        KT[s]     v[56 + 4s : +3]   K fragment temporaries (one per fragment read ahead; room for 8)
        VT[s]     v[88 + 4s : +3]   V^T fragment temporaries (one per fragment read ahead; room for 8)
        120 row max, 121 swap temp, 122 max candidate, 123 alpha, 124 max base, 125 -inf, 126..131 temps
        160..167 K fragment addresses (ks & 7), 168..175 V^T addresses (2 (dt & 3) + k-half), 176..179 own slab
        chunk addresses, 180..183 partner slab chunk addresses, 184..191 / 192..199 K / V load lane offsets,
        200 mask lane limit (Sk - 1 - 4 hf)
  AGPR  O[dt] a[16dt : +15], Q[ks] a[128 + 4ks : +3]
  SGPR  s40 tile t, s42..s43 temps, s[44:45] rescale mask, s46 tile j, s[48:51] K load
        resource, s[52:55] V load resource, s[56:63] mask compares
LDS (byte offsets from the kernel's smem, which the address operands include): K buffers 0 / 32768, V buffers
65536 / 98304 (the V^T addresses include 65536), exchange slabs 131072 / 147456 (the slab addresses include
131072).

Usage: gen_prefill_wide512.py OUT.inc -- writes DTATTN_WIDE512_PROGRAM_<BF16|F16> and DTATTN_WIDE512_CLOBBERS.
"""
import sys

NEG_FLT_MAX = "0xff7fffff"
MX, TM, MC, AL, MB, NINF, RT = 120, 121, 122, 123, 124, 125, 126
AK, AV, AS, AP, DK, DV, LIM = 160, 168, 176, 180, 184, 192, 200
NTMP = 132  # v0 .. v131 are the program's own
KBUF, VBUF_REL, SLAB_REL = 32768, 32768, 16384  # parity strides of K buffers, V buffers, slabs
SLOT_BUDGET = 30
# K and V^T fragments read ahead of their MFMAs: deeper read-ahead (6 or 8 of each) measured the same, since
# the phases are bound by LDS bandwidth rather than by the latency of one read
KAHEAD, VAHEAD = 4, 4
COST = {"v_exp_f32": 16, "v_cvt_pk_": 8}


def S(b):
    return 16 * b


def P(h):
    return 48 + 4 * h


def KT(s):
    return 56 + 4 * s  # s < 8


def VT(s):
    return 88 + 4 * s  # s < 8


def vr(r, n):
    return f"v[{r}:{r + n - 1}]"


def ar(r, n):
    return f"a[{r}:{r + n - 1}]"


def cost(ins):
    for k, v in COST.items():
        if ins.startswith(k):
            return v
    return 1 if ins.startswith("s_") else 4


class Lds:
    """In-order tracker of outstanding LDS operations: the lgkmcnt that guarantees a given one completed."""

    def __init__(self):
        self.q = []

    def issue(self, tag):
        self.q.append(tag)

    def wait_for(self, tag):
        i = self.q.index(tag)
        n = len(self.q) - 1 - i
        self.q = self.q[i + 1:]
        assert n <= 15
        return f"s_waitcnt lgkmcnt({n})"

    def drain(self):
        self.q = []


class Program:
    def __init__(self, f16):
        self.ka, self.va = KAHEAD, VAHEAD
        self.mfma = "v_mfma_f32_32x32x16_f16" if f16 else "v_mfma_f32_32x32x16_bf16"
        self.cvt = "v_cvt_pk_f16_f32" if f16 else "v_cvt_pk_bf16_f32"
        self.L = []
        self.lds = Lds()

    def e(self, *lines):
        self.L.extend(lines)

    # ---- loads ---------------------------------------------------------------------------------------
    def dma_setup(self, which, jreg):
        """Resource of tile j (SGPR jreg) of K or V: its rows below kend; none at or past the block's end."""
        pitch, rs = ("%[kp]", 48) if which == "K" else ("%[vp]", 52)
        w = which.lower()
        return [f"s_lshl_b32 s42, {jreg}, 5", f"s_mul_i32 s43, s42, {pitch}",
                f"s_add_u32 s{rs}, %[{w}lo], s43", f"s_addc_u32 s{rs + 1}, %[{w}hi], 0",
                "s_sub_i32 s43, %[kend], s42", "s_min_i32 s43, s43, 32", "s_add_i32 s43, s43, -1",
                f"s_mul_i32 s{rs + 2}, s43, {pitch}", f"s_add_i32 s{rs + 2}, s{rs + 2}, 1024",
                f"s_cmp_lt_i32 {jreg}, %[nt]", f"s_cselect_b32 s{rs + 2}, s{rs + 2}, 0",
                f"s_mov_b32 s{rs + 3}, 0x20000"]

    def dma_loads(self, which, buf):
        """This wave's 8 one-row loads of a K or V tile into buffer buf (lane l of row r0 = 8 wave + i lands at
        16 l of the row; its global chunk is l ^ wswz(r0))."""
        rs, base, off = (48, 0, DK) if which == "K" else (52, 65536, DV)
        lds = base + buf * (KBUF if which == "K" else VBUF_REL)
        return [[f"s_add_u32 m0, %[m0base], {lds + i * 1024}",
                 f"buffer_load_dwordx4 v{off + i}, s[{rs}:{rs + 3}], 0 offen lds"] for i in range(8)]

    def kread(self, kb, f):
        tag = ("K", kb, f)
        self.lds.issue(tag)
        return f"ds_read_b128 {vr(KT(f % self.ka), 4)}, v{AK + (f & 7)} offset:{kb * KBUF + 256 * (f >> 3)}"

    def vread(self, vb, m):
        ks, dt = m >> 3, m & 7
        off = vb * VBUF_REL + 16384 * ks + 256 * (dt >> 2)
        tag = ("V", vb, m)
        self.lds.issue(("V0", vb, m))
        self.lds.issue(tag)
        return [f"ds_read_b64_tr_b16 {vr(VT(m % self.va), 2)}, v{AV + 2 * (dt & 3)} offset:{off}",
                f"ds_read_b64_tr_b16 {vr(VT(m % self.va) + 2, 2)}, v{AV + 2 * (dt & 3) + 1} offset:{off}"]

    def partner_read(self, sb):
        out = []
        for j in range(4):
            self.lds.issue(("PT", j))
            out.append(f"ds_read_b128 {vr(32 + 4 * j, 4)}, v{AP + j} offset:{sb * SLAB_REL}")
        return out

    def slab_write(self, sb, b):
        out = []
        for j in range(4):
            self.lds.issue(("SW", j))
            out.append(f"ds_write_b128 v{AS + j}, {vr(S(b) + 4 * j, 4)} offset:{sb * SLAB_REL}")
        return out

    # ---- softmax pieces ------------------------------------------------------------------------------
    def softmax_valu(self, b, last):
        """Tile scores = own partial S[b] + partner PT; (last) the ragged mask; row max; the lazy-rescale
        decision (s[44:45] = all lanes when O and l must take alpha); P in place and packed to P[0..1]."""
        out = [f"v_add_f32 v{S(b) + i}, v{S(b) + i}, v{32 + i}" for i in range(16)]
        if last:
            out += self.mask_code(b)
        r = [S(b) + i for i in range(16)]
        out.append(f"v_max3_f32 v{MX}, v{r[0]}, v{r[1]}, v{r[2]}")
        for i in range(3, 15, 2):
            out.append(f"v_max3_f32 v{MX}, v{MX}, v{r[i]}, v{r[i + 1]}")
        out.append(f"v_max_f32 v{MX}, v{MX}, v{r[15]}")
        # the other half of the wave holds the same rows' other keys
        out += [f"v_mov_b32 v{TM}, v{MX}", "s_nop 1", f"v_permlane32_swap_b32 v{MX}, v{TM}",
                f"v_max_f32 v{MX}, v{MX}, v{TM}"]
        # mcand = max(m, mx c); rescale iff some row's max grew by more than 2^8; alpha = exp2(m - mcand')
        # (mcand' = 0 where mcand = -inf)
        out += [f"v_mul_f32 v{AL}, %[c], v{MX}",
                f"v_max_f32 v{MC}, %[m], v{AL}",
                f"v_sub_f32 v{AL}, v{MC}, %[m]",
                f"v_cmp_lt_f32 vcc, 0x41000000, v{AL}",
                "s_cmp_lg_u64 vcc, 0",
                "s_cselect_b64 s[44:45], exec, 0",
                f"v_cmp_eq_f32 vcc, 0xff800000, v{MC}",
                "s_nop 1",
                f"v_cndmask_b32_e64 v{AL}, v{MC}, 0, vcc",
                f"v_sub_f32 v{AL}, %[m], v{AL}",
                f"v_exp_f32 v{AL}, v{AL}",
                "s_nop 0",
                f"v_mul_f32 v{RT}, %[l], v{AL}",
                f"v_cndmask_b32_e64 %[l], %[l], v{RT}, s[44:45]",
                f"v_cndmask_b32_e64 %[m], %[m], v{MC}, s[44:45]",
                f"v_cmp_eq_f32 vcc, 0xff800000, %[m]",
                "s_nop 1",
                f"v_cndmask_b32_e64 v{MB}, %[m], 0, vcc"]
        # P = exp2(s c - mbase), summed in key order from l, packed pairwise; every exponential is read at
        # least one instruction after it is written
        fma = [f"v_fma_f32 v{x}, v{x}, %[c], -v{MB}" for x in r]
        ex = [f"v_exp_f32 v{x}, v{x}" for x in r]
        add = [f"v_add_f32 %[l], %[l], v{x}" for x in r]
        cvt = [f"{self.cvt} v{P(j // 4) + j % 4}, v{r[2 * j]}, v{r[2 * j + 1]}" for j in range(8)]
        def chain(lo, hi):
            res = []
            for st in range(lo, hi + 2):
                if st < hi:
                    res.append(fma[st])
                if lo + 1 <= st <= hi:
                    res.append(ex[st - 1])
                if st >= lo + 2:
                    res.append(add[st - 2])
                    if (st - 2) % 2 == 1:
                        res.append(cvt[(st - 2) // 2])
            return res
        if last:
            return out + chain(0, 16), []
        # the second half of P (PV k-step 1) is finished in phase B, before the MFMAs that read it
        return out + chain(0, 8), chain(8, 16)

    def mask_code(self, b):
        """Keys at or past Sk -> -inf (only a block's last tile can hold them): element i of a lane is key
        32 t + 8 (i >> 2) + 4 hf + (i & 3)."""
        out = ["s_lshl_b32 s42, s40, 5", f"v_subrev_u32 v{RT}, s42, v{LIM}"]
        offs = [(i, 8 * (i >> 2) + (i & 3)) for i in range(16)]
        for b0 in range(0, 16, 4):
            batch = offs[b0:b0 + 4]
            out += [f"v_cmp_lt_i32_e64 s[{56 + 2 * n}:{57 + 2 * n}], v{RT}, {off}" for n, (i, off) in enumerate(batch)]
            out += [f"v_cndmask_b32_e64 v{S(b) + i}, v{S(b) + i}, v{NINF}, s[{56 + 2 * n}:{57 + 2 * n}]"
                    for n, (i, off) in enumerate(batch)]
        return out

    def rescale(self, lbl):
        """O *= alpha when s[44:45] says so (wave-uniform, rare)."""
        self.e("s_cmp_eq_u64 s[44:45], 0", f"s_cbranch_scc1 {lbl}_keep")
        regs = list(range(128))
        for b0 in range(0, 128, 6):
            batch = regs[b0:b0 + 6]
            self.e(*[f"v_accvgpr_read_b32 v{RT + n}, a{a}" for n, a in enumerate(batch)])
            self.e(*[f"v_mul_f32 v{RT + n}, v{RT + n}, v{AL}" for n, a in enumerate(batch)])
            self.e(*[f"v_accvgpr_write_b32 a{a}, v{RT + n}" for n, a in enumerate(batch)])
        self.e("s_nop 2", f"{lbl}_keep:")

    @staticmethod
    def slots(valu, n=16):
        b = SLOT_BUDGET
        while True:
            out, i = [], 0
            for _ in range(n):
                sl, c = [], 0
                while i < len(valu) and (not sl or c + cost(valu[i]) <= b):
                    c += cost(valu[i])
                    sl.append(valu[i])
                    i += 1
                out.append(sl)
            if i == len(valu):
                return out
            b += 2

    # ---- phases --------------------------------------------------------------------------------------
    def phase_a(self, sn, kb, valu, dma, vpre):
        """S[sn] = K(buffer kb) Q^T, with the VALU list by slot, one load pair per MFMA (dma) and, after the last
        K reads, the first V^T reads of phase B (buffer vpre, None: none)."""
        sl = self.slots(valu)
        ka = self.ka
        self.e(*[self.kread(kb, f) for f in range(ka)])
        # V^T reads of PV MFMAs 0 .. va-1 (buffer vpre) in the slots after the last K read
        free = list(range(16 - ka, 16))
        vplan = {f: [] for f in free}
        if vpre is not None:
            for m in range(self.va):
                vplan[free[m * len(free) // self.va]].append(m)
        for f in range(16):
            self.e(self.lds.wait_for(("K", kb, f)))
            d = vr(S(sn), 16)
            self.e(f"{self.mfma} {d}, {vr(KT(f % ka), 4)}, {ar(128 + 4 * f, 4)}, {'0' if f == 0 else d}")
            if f + ka < 16:
                self.e(self.kread(kb, f + ka))
            else:
                for m in vplan[f]:
                    self.e(*self.vread(vpre, m))
            if dma and f < len(dma):
                self.e(*dma[f])
            self.e(*sl[f])

    def phase_b(self, vb, slab, dma=None, valu=()):
        """O^T += V(buffer vb)^T P^T, with one load pair per MFMA (dma) and VALU (the second half of P) in the
        first six slots, two MFMAs ahead of the k-step that reads it; then (slab = (parity, S buffer)) this
        wave's partial into the slab."""
        sl = self.slots(list(valu), 6) + [[] for _ in range(10)] if valu else [[] for _ in range(16)]
        for m in range(16):
            ks, dt = m >> 3, m & 7
            self.e(self.lds.wait_for(("V", vb, m)))
            o = ar(16 * dt, 16)
            self.e(f"{self.mfma} {o}, {vr(VT(m % self.va), 4)}, {vr(P(ks), 4)}, {o}")
            if m + self.va < 16:
                self.e(*self.vread(vb, m + self.va))
            if dma and m < len(dma):
                self.e(*dma[m])
            self.e(*sl[m])
            if m == 12 and slab is not None:
                self.e(*self.slab_write(*slab))

    def step_end(self):
        self.e("s_waitcnt vmcnt(0) lgkmcnt(0)", "s_barrier")
        self.lds.drain()

    # ---- the loop ----------------------------------------------------------------------------------
    def step(self, par, u):
        """Tile t = s40 of parity par: its own partial in S[par], partials in slab par, K(t+1) in K buffer 1-par,
        V(t) in V buffer par.  Computes S(t+1) -> S[1-par] and slab 1-par; loads K(t+2) -> K buffer par and
        V(t+1) -> V buffer 1-par."""
        lb = f"L{u}_%="
        self.e("s_add_i32 s46, s40, 1", "s_cmp_lt_i32 s46, %[nt]", f"s_cbranch_scc0 {lb}_last")
        self.e(*self.dma_setup("V", "s46"), "s_add_i32 s46, s40, 2", *self.dma_setup("K", "s46"))
        self.e(*self.partner_read(par))
        va, vb = self.softmax_valu(par, False)
        self.phase_a(1 - par, 1 - par, va, self.dma_loads("K", par), par)
        self.rescale(f"{lb}_r")
        self.phase_b(par, (1 - par, 1 - par), self.dma_loads("V", 1 - par), vb)
        self.step_end()
        self.e(f"s_branch {lb}_next", f"{lb}_last:")
        # a block's last tile: no next scores, no loads
        self.lds.drain()
        self.e(*self.partner_read(par))
        self.e(self.lds.wait_for(("PT", 3)))
        self.e(*self.softmax_valu(par, True)[0])
        self.rescale(f"{lb}_q")
        self.e(*[x for m in range(self.va) for x in self.vread(par, m)])
        self.phase_b(par, None)
        self.step_end()
        self.e(f"{lb}_next:", "s_add_i32 s40, s40, 1")

    def program(self):
        self.e(f"v_mov_b32 v{NINF}, 0xff800000", "s_mov_b32 s40, %[t0]")
        # S(t0) -> S[0] and slab 0 from K buffer 0 (tile t0 is in place), with K(t0+1) -> K buffer 1
        self.e("s_add_i32 s46, s40, 1", *self.dma_setup("K", "s46"))
        self.phase_a(0, 0, [], self.dma_loads("K", 1), None)
        self.e("s_nop 7", "s_nop 7", "s_nop 4", *self.slab_write(0, 0))
        self.step_end()
        self.e("L_top_%=:")
        self.step(0, "e")
        self.e("s_cmp_lt_i32 s40, %[nt]", "s_cbranch_scc0 L_end_%=")
        self.step(1, "o")
        self.e("s_cmp_lt_i32 s40, %[nt]", "s_cbranch_scc1 L_top_%=", "L_end_%=:")
        # the last PV MFMAs' results need their wait states before the compiler's code reads O
        self.e("s_nop 7", "s_nop 7", "s_nop 4")
        return self.L


def main(path):
    out = ["// Generated by gen_prefill_wide512.py: do not edit.\n#pragma once\n"]
    for f16 in (False, True):
        lines = Program(f16).program()
        out.append(f"#define DTATTN_WIDE512_PROGRAM_{'F16' if f16 else 'BF16'} \\")
        out.append(" \\\n".join('    "' + l + '\\n"' for l in lines))
        out.append("")
    clob = ", ".join(f'"v{i}"' for i in range(NTMP)) + ", " + ", ".join(f'"s{i}"' for i in range(40, 64))
    out.append(f'#define DTATTN_WIDE512_CLOBBERS {clob}, "vcc", "m0", "memory"')
    tmp = path + ".tmp"
    with open(tmp, "w") as fh:
        fh.write("\n".join(out) + "\n")
    import os
    os.replace(tmp, path)


if __name__ == "__main__":
    main(sys.argv[1])
