"""Generator of the pipelined forward kernel's inline assembly (bsa_pipe_asm.inc).

The kernel bsa_fwd_pipe_kernel<kRows> (bsa_fwd.hip) runs one (b*h, query block) work item per
256-thread workgroup, two workgroups per CU, each wave owning 32 query rows, like
bsa_fwd_dma_kernel. What differs is the schedule of a work item's key blocks b_0 (the diagonal),
b_1 .. b_n (the off-diagonal entries): iteration i (0 <= i < n) runs, in four slots t = 0..3,

    S^T(b_{i+1}, key tile t) = K · Q^T           8 MFMAs, K sub-tile t from LDS
    O^T += V^T(b_i, keys 32t..32t+31) · P^T       8 MFMAs, V sub-tile t from LDS
    one key tile's softmax (slot 0: tile 3 of b_i, slot t > 0: tile t-1 of b_{i+1})

interleaved instruction by instruction, so every wave keeps the matrix core, the VALU and the
LDS busy together instead of alternating an MFMA phase and a softmax phase. K and V move through
LDS in 8 KiB sub-tiles (32 keys): the barrier that opens slot t releases sub-tile t-1 of both
tiles, whose refills (K of b_{i+2}, V of b_{i+1}) are issued right after it and used three slots
later. The diagonal block b_0 is computed before the loop with its exact row max; a last pass
runs P·V of b_n. P of the off-diagonal blocks uses the running row max as it stands and is
accepted when the fp32 row sum of its tiles is <= 2^12 (tiles 0-2 checked at the end of the
iteration that computed them, tile 3 before its P·V); otherwise an out-of-line block moves the
row max to the exact one, rescales O and l and recomputes the affected P tiles.

Everything of a work item after the C++ prologue (item coordinates, CSR row bounds) is one asm
statement: Q loads, tile DMAs, MFMAs, softmax, O through LDS to HBM and the LSE. Registers are
fixed (S v0-63, P v64-95, Q v96-127, operand rings, softmax temporaries, row state; O in
a0-a63); per-lane addresses come in as "v" operands and uniform values as "s" operands.

The generator keeps track of the gfx950 hazards the hardware does not check (an MFMA result read
by a non-MFMA instruction: 12 wait states; a VALU result read by an MFMA: 2; v_exp_f32 result by
a VALU: 1; a VALU result by v_permlane32_swap: 2; an SGPR written by SALU read by a memory
instruction: 1, by VALU: 5) and inserts s_nop where the instruction stream does not already
space them; LDS and global load results are waited for with counted s_waitcnt.

usagi_amd/build.py runs it before every compile (python3 usagi_amd/csrc/gen_bsa_pipe.py writes
bsa_pipe_asm.inc next to this file; --check compares an existing file with its output).
"""
from __future__ import annotations

import os
import re
import sys

# ------------------------------------------------------------------------------------------
# register map (per wave)
# ------------------------------------------------------------------------------------------


def S(t):  # S^T key tile t (keys 32t..32t+31): 16 accumulators
    return 16 * t


def P(ks):  # P k-step ks (keys 16ks..16ks+15) in fp16: 4 dwords
    return 64 + 4 * ks


def Q(s):  # Q operand for head-dim step s (d = 16s..16s+15): 4 dwords
    return 96 + 4 * s


D = 2  # operand read-ahead (ring slots per operand kind)
KR = 128  # K operand ring: D x 4
VR = 136  # V operand ring: D x 4
TMP = 144  # 8 softmax temporaries v144..v151
M = 152  # running row max (scaled, base-2 units)
LACC = 153  # committed row sum (this lane's keys)
LPEND = 154  # sum of the key tiles computed ahead (tiles 0-2 of the next block)
LT3 = 155  # sum of key tile 3 of the block being multiplied
DUMMY = 156  # target of placeholder loads
T2 = 157  # v157..v163: spare temporaries
NEGINF = 163
KA = 164  # v164..v171: K operand read address for head-dim step s (LDS, row li, swizzled)
VA = 172  # v172..v175: V^T operand read address for d group u (LDS)
LAST_V = 175
N_AGPR = 64

# scratch SGPRs (clobbered)
SI = 60  # iteration i
ST = 61  # temporary
SP = 62  # s[62:63] DMA source pair
KBA = 64  # s[64:65] K base of b_{i+1}
KBB = 66  # s[66:67] K base of b_{i+2}
VBA = 68  # s[68:69] V base of b_i
VBB = 70  # s[70:71] V base of b_{i+1}
VBC = 72  # s[72:73] V base of b_{i+2}
SX = 74  # s[74:75] misc pair (Q, O, LSE bases)
SE = 76  # entry index
SKB = 77  # key block of a lookup
SREAL = 78  # 1 when b_{i+2} exists
ST2 = 79
SCB = 80  # s[80:81] column list base (CSR)
KHB = 84  # s[84:85] K of this (b, h)
VHB = 86  # s[86:87] V of this (b, h)
KL = 88  # LDS: K buffer + 2048 * wave (this wave's DMA rows of a sub-tile)
VL = 89  # LDS: V buffer + 2048 * wave
STG = 90  # LDS: K buffer + 8192 * wave (O staging)
SGPR_LO, SGPR_HI = 60, 90

NEG_INF_BITS = "0xff800000"
SPEC_SUM = "0x45800000"  # 4096.0: acceptance bound of a speculative row sum

# ------------------------------------------------------------------------------------------
# emitter
# ------------------------------------------------------------------------------------------


def vr(lo, n=1):
    return [f"v{i}" for i in range(lo, lo + n)]


def ar(lo, n=1):
    return [f"a{i}" for i in range(lo, lo + n)]


def sr(lo, n=1):
    return [f"s{i}" for i in range(lo, lo + n)]


def vrange(lo, n):
    return f"v{lo}" if n == 1 else f"v[{lo}:{lo + n - 1}]"


def arange_(lo, n):
    return f"a{lo}" if n == 1 else f"a[{lo}:{lo + n - 1}]"


class Em:
    MFMA_OTHER = 12
    VALU_MFMA = 2
    TRANS_VALU = 1
    VALU_PERM = 2
    VALU_SGPR_USE = 5
    SALU_MEM = 1

    def __init__(self):
        self.out = []
        self.t = 0
        self.last_w = {}
        self.lgkm = []  # outstanding LDS reads: sets of destination registers, in issue order
        self.vm = []  # outstanding global loads / DMAs: sets of destination registers

    def snapshot(self):
        return (self.t, dict(self.last_w), list(self.lgkm), list(self.vm))

    def restore(self, snap):
        self.t, lw, lg, vm = snap
        self.last_w, self.lgkm, self.vm = dict(lw), list(lg), list(vm)

    def raw(self, text):
        self.out.append(text)
        m = re.match(r"s_nop (\d+)", text)
        self.t += int(m.group(1)) + 1 if m else 1

    def nops(self, n):
        while n > 0:
            k = min(n, 8)
            self.raw(f"s_nop {k - 1}")
            n -= k

    def label(self, name, settle=True):
        """A branch target. settle: pad so that no hazard of any path into it can remain."""
        self.out.append(f"{name}:")
        if settle:
            self.nops(self.MFMA_OTHER)
            self.last_w = {}

    def _need(self, cls, reads, writes):
        need = 0
        for r in reads | writes:
            if r not in self.last_w:
                continue
            tw, wc = self.last_w[r]
            since = self.t - tw - 1  # wait states issued since the writer
            req = 0
            if wc == "mfma":
                if cls != "mfma":
                    req = self.MFMA_OTHER
            elif wc in ("valu", "trans", "perm", "readlane"):
                if cls == "mfma" and r in reads:
                    req = self.VALU_MFMA
                if wc == "trans" and cls in ("valu", "trans", "perm") and r in reads:
                    req = max(req, self.TRANS_VALU)
                if cls == "perm" and r in reads:
                    req = max(req, self.VALU_PERM)
                if r.startswith("s") and r in reads and cls not in ("salu",):
                    req = max(req, self.VALU_SGPR_USE)
            elif wc == "salu":
                if cls in ("vmem", "dma", "ds") and r in reads:
                    req = self.SALU_MEM
            need = max(need, req - since)
        return need

    def _wait_queue(self, q, regs, kind, limit):
        idx = -1
        for i, ws in enumerate(q):
            if ws & regs:
                idx = i
        if idx < 0:
            return q
        n = len(q) - idx - 1
        assert n <= limit, (kind, n)
        self.raw(f"s_waitcnt {kind}({n})")
        return q[idx + 1:]

    def emit(self, cls, text, reads=(), writes=()):
        reads, writes = set(reads), set(writes)
        self.lgkm = self._wait_queue(self.lgkm, reads | writes, "lgkmcnt", 15)
        self.vm = self._wait_queue(self.vm, reads | writes, "vmcnt", 63)
        self.nops(self._need(cls, reads, writes))
        self.out.append(text)
        self.t += 1
        for r in writes:
            self.last_w[r] = (self.t - 1, cls)
        if cls == "ds":
            self.lgkm.append(set(writes))
        elif cls in ("vmem", "dma"):
            self.vm.append(set(writes))

    def wait_vm(self, n):
        self.raw(f"s_waitcnt vmcnt({n})")
        if len(self.vm) > n:
            self.vm = self.vm[len(self.vm) - n:] if n else []

    def wait_lgkm0(self):
        if self.lgkm:
            self.raw("s_waitcnt lgkmcnt(0)")
            self.lgkm = []

    def barrier(self):
        self.wait_lgkm0()
        self.raw("s_barrier")


# ------------------------------------------------------------------------------------------
# building blocks
# ------------------------------------------------------------------------------------------

IN = "%[{}]"  # asm operand reference


def inp(name):
    return IN.format(name)


def softmax_ops(t, sum_reg):
    """VALU ops of one key tile's softmax: P = exp2(S * scale - m) in fp16 (P k-steps 2t, 2t+1)
    and its fp32 row sum added to sum_reg. Element r of tile t is key 32t + 8(r/4) + 4(l/32) +
    r%4; P k-step ks dword d packs elements 8(ks%2) + 2d and +1 (the MFMA B-operand order)."""
    ops = []
    sc = inp("scale")
    for pr in range(8):
        r0, r1 = 2 * pr, 2 * pr + 1
        t0, t1 = TMP + (2 * pr) % 8, TMP + (2 * pr + 1) % 8
        ks = 2 * t + (1 if r0 >= 8 else 0)
        d = (r0 % 8) // 2
        ops.append(("valu", f"v_fma_f32 v{t0}, v{S(t) + r0}, {sc}, -v{M}", vr(S(t) + r0) + vr(M), vr(t0)))
        ops.append(("valu", f"v_fma_f32 v{t1}, v{S(t) + r1}, {sc}, -v{M}", vr(S(t) + r1) + vr(M), vr(t1)))
        ops.append(("trans", f"v_exp_f32 v{t0}, v{t0}", vr(t0), vr(t0)))
        ops.append(("trans", f"v_exp_f32 v{t1}, v{t1}", vr(t1), vr(t1)))
        ops.append(("valu", f"v_add_f32 v{sum_reg}, v{sum_reg}, v{t0}", vr(sum_reg) + vr(t0), vr(sum_reg)))
        ops.append(("valu", f"v_add_f32 v{sum_reg}, v{sum_reg}, v{t1}", vr(sum_reg) + vr(t1), vr(sum_reg)))
        ops.append(("valu", f"v_cvt_pk_f16_f32 v{P(ks) + d}, v{t0}, v{t1}", vr(t0) + vr(t1), vr(P(ks) + d)))
    return ops


def emit_ops(em, ops):
    for op in ops:
        em.emit(*op)


def dma_ops(tile_pair, sub, lds_name, offs):
    """DMA of this wave's two 1 KiB pieces of sub-tile `sub` (rows 32sub + 8w + 4i + L/16) from
    the tile whose base is in s[tile_pair:tile_pair+1] into LDS (K or V buffer + 2048 w)."""
    ops = [
        ("salu", f"s_add_u32 s{SP}, s{tile_pair}, {sub * 8192}", sr(tile_pair), sr(SP) + ["scc"]),
        ("salu", f"s_addc_u32 s{SP + 1}, s{tile_pair + 1}, 0", sr(tile_pair + 1) + ["scc"], sr(SP + 1) + ["scc"]),
        ("salu", f"s_add_u32 m0, s{lds_name}, {sub * 8192}", sr(lds_name), ["m0", "scc"]),
    ]
    for i in range(2):
        ops.append(("dma", f"global_load_lds_dwordx4 {inp(offs[i])}, s[{SP}:{SP + 1}] offset:{1024 * i}",
                    sr(SP, 2) + ["m0"], []))
    return ops


def dummy_ops():
    """Two placeholder loads (in place of a DMA pair that has no tile to move), so that every
    path issues the same number of memory operations and the vmcnt waits stay exact."""
    return [("vmem", f"global_load_dword v{DUMMY}, {inp('qo')}, s[{KHB}:{KHB + 1}]", sr(KHB, 2), [])] * 2


def kb_lookup(mode, e_reg, kdst, vdst):
    """SALU (+ one v_readlane for CSR rows): K and V tile bases of off-diagonal entry e."""
    ops = []
    if mode == "csr":
        ops.append(("salu", f"s_and_b32 s{ST2}, s{e_reg}, 63", sr(e_reg), sr(ST2) + ["scc"]))
        ops.append(("readlane", f"v_readlane_b32 s{SKB}, {inp('colv')}, s{ST2}", sr(ST2), sr(SKB)))
        ops.append(("salu", f"s_max_i32 s{SKB}, s{SKB}, 0", sr(SKB), sr(SKB) + ["scc"]))
        ops.append(("salu", f"s_min_i32 s{SKB}, s{SKB}, {inp('nqm1')}", sr(SKB), sr(SKB) + ["scc"]))
    else:
        ops.append(("salu", f"s_sub_i32 s{SKB}, s{e_reg}, {inp('wng')}", sr(e_reg), sr(SKB) + ["scc"]))
        ops.append(("salu", f"s_add_i32 s{SKB}, s{SKB}, {inp('wlo')}", sr(SKB), sr(SKB) + ["scc"]))
        ops.append(("salu", f"s_cmp_lt_i32 s{e_reg}, {inp('wng')}", sr(e_reg), ["scc"]))
        ops.append(("salu", f"s_cselect_b32 s{SKB}, s{e_reg}, s{SKB}", sr(e_reg) + sr(SKB) + ["scc"], sr(SKB)))
    ops += tile_bases(SKB, kdst, vdst)
    return ops


def tile_bases(kb_reg, kdst, vdst):
    return [
        ("salu", f"s_lshl_b32 s{ST2}, s{kb_reg}, 15", sr(kb_reg), sr(ST2) + ["scc"]),
        ("salu", f"s_add_u32 s{kdst}, s{KHB}, s{ST2}", sr(ST2) + sr(KHB), sr(kdst) + ["scc"]),
        ("salu", f"s_addc_u32 s{kdst + 1}, s{KHB + 1}, 0", ["scc"] + sr(KHB + 1), sr(kdst + 1) + ["scc"]),
        ("salu", f"s_add_u32 s{vdst}, s{VHB}, s{ST2}", sr(ST2) + sr(VHB), sr(vdst) + ["scc"]),
        ("salu", f"s_addc_u32 s{vdst + 1}, s{VHB + 1}, 0", ["scc"] + sr(VHB + 1), sr(vdst + 1) + ["scc"]),
    ]


def pair_reduce(em, x, op):
    """x = op(x[l], x[l ^ 32]) across the two lanes of a query row."""
    a, b = T2, T2 + 1
    em.emit("valu", f"v_mov_b32 v{a}, v{x}", vr(x), vr(a))
    em.emit("valu", f"v_mov_b32 v{b}, v{x}", vr(x), vr(b))
    em.emit("perm", f"v_permlane32_swap_b32 v{a}, v{b}", vr(a, 1) + vr(b, 1), vr(a) + vr(b))
    em.emit("valu", f"{op} v{x}, v{a}, v{b}", vr(a) + vr(b), vr(x))


def row_max(em, tiles, dst):
    """dst = max over the given key tiles of this lane's S (v_max3 chain)."""
    regs = [S(t) + r for t in tiles for r in range(16)]
    em.emit("valu", f"v_max3_f32 v{dst}, v{regs[0]}, v{regs[1]}, v{regs[2]}", vr(regs[0]) + vr(regs[1]) + vr(regs[2]), vr(dst))
    rest = regs[3:]
    while rest:
        if len(rest) >= 2:
            em.emit("valu", f"v_max3_f32 v{dst}, v{dst}, v{rest[0]}, v{rest[1]}", vr(dst) + vr(rest[0]) + vr(rest[1]), vr(dst))
            rest = rest[2:]
        else:
            em.emit("valu", f"v_max_f32 v{dst}, v{dst}, v{rest[0]}", vr(dst) + vr(rest[0]), vr(dst))
            rest = rest[1:]


def rescale_to(em, tiles):
    """Move the row max to max(m, exact max of the given S tiles * scale); rescale l and O."""
    mx, alpha = T2 + 2, T2 + 3
    row_max(em, tiles, mx)
    pair_reduce(em, mx, "v_max_f32")
    em.emit("valu", f"v_mul_f32 v{mx}, {inp('scale')}, v{mx}", vr(mx), vr(mx))
    em.emit("valu", f"v_max_f32 v{mx}, v{M}, v{mx}", vr(M) + vr(mx), vr(mx))
    em.emit("valu", f"v_sub_f32 v{alpha}, v{M}, v{mx}", vr(M) + vr(mx), vr(alpha))
    em.emit("trans", f"v_exp_f32 v{alpha}, v{alpha}", vr(alpha), vr(alpha))
    em.emit("valu", f"v_mov_b32 v{M}, v{mx}", vr(mx), vr(M))
    em.emit("valu", f"v_mul_f32 v{LACC}, v{LACC}, v{alpha}", vr(LACC) + vr(alpha), vr(LACC))
    # O *= alpha through VGPR temporaries, 8 at a time
    tmps = list(range(TMP, TMP + 8))
    for base in range(0, N_AGPR, 8):
        for k in range(8):
            em.emit("valu", f"v_accvgpr_read_b32 v{tmps[k]}, a{base + k}", ar(base + k), vr(tmps[k]))
        for k in range(8):
            em.emit("valu", f"v_mul_f32 v{tmps[k]}, v{tmps[k]}, v{alpha}", vr(tmps[k]) + vr(alpha), vr(tmps[k]))
        for k in range(8):
            em.emit("valu", f"v_accvgpr_write_b32 a{base + k}, v{tmps[k]}", vr(tmps[k]), ar(base + k))


# ------------------------------------------------------------------------------------------
# the work item
# ------------------------------------------------------------------------------------------


class Kernel:
    def __init__(self, mode, bf16=False):
        assert mode in ("csr", "window")
        self.mode = mode
        self.bf16 = bf16
        # Q·K^T in the input type; P·V always in fp16 (bf16 V is turned into fp16 in LDS)
        self.qk_op = "v_mfma_f32_32x32x16_bf16" if bf16 else "v_mfma_f32_32x32x16_f16"
        self.em = Em()
        self.ool = []  # out-of-line blocks (fallbacks), appended after the epilogue

    def L(self, name):
        return f".Lbsa_{name}_%="

    # ---- one slot of a pipelined pass -------------------------------------------------------
    def slot(self, t, *, qk, sm, sm_sum, vmwait, k_refill, v_refill, pre=(), side=()):
        """qk: run Q·K^T of the next block on key tile t. sm: key tile whose softmax runs here
        (or None). k_refill: "real" / "branch" / None; v_refill: tile-base pair or None.
        vmwait: int, or (count at i == 0, count otherwise)."""
        em = self.em
        em.wait_lgkm0()
        if isinstance(vmwait, tuple):
            first, other = vmwait
            lo, done = self.L(f"w{t}o"), self.L(f"w{t}d")
            em.raw(f"s_cmp_eq_u32 s{SI}, 0")
            em.raw(f"s_cbranch_scc0 {lo}")
            em.raw(f"s_waitcnt vmcnt({first})")
            em.raw(f"s_branch {done}")
            em.out.append(f"{lo}:")
            em.raw(f"s_waitcnt vmcnt({other})")
            em.out.append(f"{done}:")
            em.vm = []
        else:
            em.wait_vm(vmwait)
            em.vm = []
        for op in pre:
            em.emit(*op)
        if self.bf16:
            self.convert_v(t)
        em.barrier()
        # MFMAs of the slot: Q·K^T steps and P·V (k-steps 2t, 2t+1) alternating
        qks = [("qk", s) for s in range(8)] if qk else []
        pvs = [("pv", ks, u) for ks in (2 * t, 2 * t + 1) for u in range(4)]
        mf = []
        for i in range(max(len(qks), len(pvs))):
            if i < len(qks):
                mf.append(qks[i])
            if i < len(pvs):
                mf.append(pvs[i])
        kq = [m for m in mf if m[0] == "qk"]
        vq = [m for m in mf if m[0] == "pv"]
        state = {"nk": 0, "nv": 0}

        def read_k(i):
            s = kq[i][1]
            b = KR + 4 * (i % D)
            em.emit("ds", f"ds_read_b128 v[{b}:{b + 3}], v{KA + s} offset:{t * 8192}", vr(KA + s), vr(b, 4))

        def read_v(i):
            _, ks, u = vq[i]
            b = VR + 4 * (i % D)
            em.emit("ds", f"ds_read_b64_tr_b16 v[{b}:{b + 1}], v{VA + u} offset:{ks * 4096}", vr(VA + u), vr(b, 2))
            em.emit("ds", f"ds_read_b64_tr_b16 v[{b + 2}:{b + 3}], v{VA + u} offset:{ks * 4096 + 2048}", vr(VA + u), vr(b + 2, 2))

        for i in range(min(D - 1, len(kq))):
            read_k(i)
            state["nk"] += 1
        for i in range(min(D - 1, len(vq))):
            read_v(i)
            state["nv"] += 1
        # side work spread over the MFMAs: refill DMAs first, then other groups, then softmax
        sub = (t - 1) % 4
        groups = []
        if k_refill == "branch":
            groups.append(("kbranch", sub))
        elif k_refill is not None:
            groups.append(("ops", dma_ops(KBA if t == 0 else KBB, sub, KL, ("ko0", "ko1"))))
        if v_refill is not None:
            groups.append(("ops", dma_ops(v_refill, sub, VL, ("vo", "vo"))))
        for g in side:
            groups.append(("ops", list(g)))
        smx = softmax_ops(sm, sm_sum) if sm is not None else []
        n = len(mf)
        per = [[] for _ in range(n)]
        for gi, g in enumerate(groups):
            per[min(gi + 1, n - 1)].append(g)
        for i, op in enumerate(smx):
            per[1 + (i * (n - 1)) // len(smx)].append(("ops", [op]))
        for i, m in enumerate(mf):
            if m[0] == "qk":
                ki = kq.index(m)
                if state["nk"] < len(kq) and state["nk"] <= ki + D - 1:
                    read_k(state["nk"])
                    state["nk"] += 1
                s = m[1]
                b = KR + 4 * (ki % D)
                c = "0" if s == 0 else vrange(S(t), 16)
                rd = vr(b, 4) + vr(Q(s), 4) + ([] if s == 0 else vr(S(t), 16))
                em.emit("mfma", f"{self.qk_op} {vrange(S(t), 16)}, v[{b}:{b + 3}], v[{Q(s)}:{Q(s) + 3}], {c}",
                        rd, vr(S(t), 16))
            else:
                vi = vq.index(m)
                if state["nv"] < len(vq) and state["nv"] <= vi + D - 1:
                    read_v(state["nv"])
                    state["nv"] += 1
                _, ks, u = m
                b = VR + 4 * (vi % D)
                em.emit("mfma", f"v_mfma_f32_32x32x16_f16 {arange_(16 * u, 16)}, v[{b}:{b + 3}], v[{P(ks)}:{P(ks) + 3}], {arange_(16 * u, 16)}",
                        vr(b, 4) + vr(P(ks), 4) + ar(16 * u, 16), ar(16 * u, 16))
            for kind, arg in per[i]:
                if kind == "ops":
                    emit_ops(em, arg)
                else:
                    self.k_refill_branch(t, arg)
        em.wait_lgkm0()

    def convert_v(self, t):
        """bf16 inputs: this wave's two 1 KiB pieces of V sub-tile t (the rows its DMA wrote) are
        turned into fp16 in place after they land and before the barrier that opens slot t, so
        P·V runs on fp16 V as the reference's does. Each dword of two bf16 widens exactly to two
        fp32 (a shift and a mask) and is packed to fp16 by one v_cvt_pk_f16_f32."""
        em = self.em
        a, lo, hi = T2 + 5, T2 + 3, T2 + 4
        em.emit("valu", f"v_lshlrev_b32 v{a}, 4, {inp('lid')}", [], vr(a))
        em.emit("valu", f"v_add_u32 v{a}, s{VL}, v{a}", vr(a) + sr(VL), vr(a))
        for i in range(2):
            em.emit("ds", f"ds_read_b128 v[{TMP + 4 * i}:{TMP + 4 * i + 3}], v{a} offset:{t * 8192 + 1024 * i}",
                    vr(a), vr(TMP + 4 * i, 4))
        for j in range(8):
            d = TMP + j
            em.emit("valu", f"v_lshlrev_b32 v{lo}, 16, v{d}", vr(d), vr(lo))
            em.emit("valu", f"v_and_b32 v{hi}, 0xffff0000, v{d}", vr(d), vr(hi))
            em.emit("valu", f"v_cvt_pk_f16_f32 v{d}, v{lo}, v{hi}", vr(lo) + vr(hi), vr(d))
        for i in range(2):
            em.emit("dsw", f"ds_write_b128 v{a}, v[{TMP + 4 * i}:{TMP + 4 * i + 3}] offset:{t * 8192 + 1024 * i}",
                    vr(a) + vr(TMP + 4 * i, 4), [])
        em.raw("s_waitcnt lgkmcnt(0)")

    def k_refill_branch(self, t, sub):
        """K(b_{i+2}, sub) refill when b_{i+2} exists, placeholder loads otherwise."""
        em = self.em
        dmy, done = self.L(f"kd{t}"), self.L(f"kj{t}")
        em.raw(f"s_cmp_eq_u32 s{SREAL}, 0")
        em.raw(f"s_cbranch_scc1 {dmy}")
        snap = em.snapshot()
        emit_ops(em, dma_ops(KBB, sub, KL, ("ko0", "ko1")))
        em.raw(f"s_branch {done}")
        t_real = em.t
        em.restore(snap)
        em.out.append(f"{dmy}:")
        emit_ops(em, dummy_ops())
        em.out.append(f"{done}:")
        em.t = max(em.t, t_real)

    # ---- prologue: Q, diagonal block --------------------------------------------------------
    def prologue(self):
        em = self.em
        # lane values: li = lid & 31, dlim = li - 4 (lid >> 5)
        li, lh4, dlim = T2, T2 + 1, T2 + 2
        em.emit("valu", f"v_and_b32 v{li}, 31, {inp('lid')}", [], vr(li))
        em.emit("valu", f"v_lshrrev_b32 v{lh4}, 5, {inp('lid')}", [], vr(lh4))
        em.emit("valu", f"v_lshlrev_b32 v{lh4}, 2, v{lh4}", vr(lh4), vr(lh4))
        em.emit("valu", f"v_sub_u32 v{dlim}, v{li}, v{lh4}", vr(li) + vr(lh4), vr(dlim))
        em.emit("valu", f"v_mov_b32 v{NEGINF}, {NEG_INF_BITS}", [], vr(NEGINF))
        # K / V operand read addresses: K row li, chunk (2s + lh) ^ (li & 15) -> krow + (32 s ^ kx);
        # V^T reads: vrow + (64 u ^ 64 tq)
        for s_ in range(8):
            em.emit("valu", f"v_xor_b32 v{KA + s_}, {32 * s_}, {inp('kx')}", [], vr(KA + s_))
            em.emit("valu", f"v_add_u32 v{KA + s_}, {inp('krow')}, v{KA + s_}", vr(KA + s_), vr(KA + s_))
        for u in range(4):
            em.emit("valu", f"v_xor_b32 v{VA + u}, {64 * u}, {inp('tq')}", [], vr(VA + u))
            em.emit("valu", f"v_add_u32 v{VA + u}, {inp('vrow')}, v{VA + u}", vr(VA + u), vr(VA + u))
        em.emit("salu", f"s_mov_b64 s[{KHB}:{KHB + 1}], {inp('kb')}", [], sr(KHB, 2))
        em.emit("salu", f"s_mov_b64 s[{VHB}:{VHB + 1}], {inp('vb')}", [], sr(VHB, 2))
        em.emit("salu", f"s_lshl_b32 s{ST}, {inp('wave')}, 11", [], sr(ST) + ["scc"])
        em.emit("salu", f"s_add_u32 s{KL}, {inp('klds')}, s{ST}", sr(ST), sr(KL) + ["scc"])
        em.emit("salu", f"s_add_u32 s{VL}, {inp('vlds')}, s{ST}", sr(ST), sr(VL) + ["scc"])
        em.emit("salu", f"s_lshl_b32 s{ST}, {inp('wave')}, 13", [], sr(ST) + ["scc"])
        em.emit("salu", f"s_add_u32 s{STG}, {inp('klds')}, s{ST}", sr(ST), sr(STG) + ["scc"])
        for r in (M, LACC, LPEND, LT3):
            em.emit("valu", f"v_mov_b32 v{r}, 0", [], vr(r))
        # Q rows of this wave: 8 x 16 bytes per lane
        em.emit("salu", f"s_mov_b64 s[{SX}:{SX + 1}], {inp('q')}", [], sr(SX, 2))
        for s in range(8):
            em.emit("vmem", f"global_load_dwordx4 v[{Q(s)}:{Q(s) + 3}], {inp('qo')}, s[{SX}:{SX + 1}] offset:{32 * s}",
                    sr(SX, 2), vr(Q(s), 4))
        # O accumulators start at zero (every P·V MFMA accumulates)
        for r in range(N_AGPR):
            em.emit("valu", f"v_accvgpr_write_b32 a{r}, 0", [], ar(r))
        # tile bases: b_0 = qb -> (KBA, VBA); b_1 = entry 0 -> (KBB, VBB)
        emit_ops(em, [("salu", f"s_mov_b32 s{SKB}, {inp('qblk')}", [], sr(SKB))])
        emit_ops(em, tile_bases(SKB, KBA, VBA))
        em.emit("salu", f"s_mov_b32 s{SE}, 0", [], sr(SE))
        emit_ops(em, kb_lookup(self.mode, SE, KBB, VBB))
        # K(b_0) whole tile, V(b_0) sub-tiles 0-2
        for sub in range(4):
            emit_ops(em, dma_ops(KBA, sub, KL, ("ko0", "ko1")))
        for sub in range(3):
            emit_ops(em, dma_ops(VBA, sub, VL, ("vo", "vo")))
        em.wait_vm(6)  # Q and K(b_0) have landed (V(b_0) may still be in flight)
        em.barrier()
        # diagonal Q·K^T: wave w needs key tiles 0..w
        join = self.L("diag_join")
        labels = [self.L(f"diag{w}") for w in range(4)]
        for w in range(3):
            em.raw(f"s_cmp_eq_u32 {inp('wave')}, {w}")
            em.raw(f"s_cbranch_scc1 {labels[w]}")
        em.raw(f"s_branch {labels[3]}")
        snap = em.snapshot()
        t_max = em.t
        for w in range(4):
            em.restore(snap)
            em.out.append(f"{labels[w]}:")
            self.diag_wave(w, dlim)
            em.raw(f"s_branch {join}")
            t_max = max(t_max, em.t)
        em.label(join)
        em.t = max(em.t, t_max)

    def diag_wave(self, w, dlim):
        em = self.em
        # Q·K^T on key tiles 0..w (K operands D ahead)
        ops = [(t, s) for t in range(w + 1) for s in range(8)]
        ring = {}

        def rd(i):
            t, s = ops[i]
            b = KR + 4 * (i % D)
            em.emit("ds", f"ds_read_b128 v[{b}:{b + 3}], v{KA + s} offset:{t * 8192}", vr(KA + s), vr(b, 4))
            ring[i] = b

        for i in range(min(D, len(ops))):
            rd(i)
        for i, (t, s) in enumerate(ops):
            b = ring[i]
            c = "0" if s == 0 else vrange(S(t), 16)
            rdregs = vr(b, 4) + vr(Q(s), 4) + ([] if s == 0 else vr(S(t), 16))
            em.emit("mfma", f"{self.qk_op} {vrange(S(t), 16)}, v[{b}:{b + 3}], v[{Q(s)}:{Q(s) + 3}], {c}",
                    rdregs, vr(S(t), 16))
            if i + D < len(ops):
                rd(i + D)
        em.wait_lgkm0()
        # tiles above the wave's rows: S = -inf (their P is 0)
        for t in range(w + 1, 4):
            for r in range(16):
                em.emit("valu", f"v_mov_b32 v{S(t) + r}, v{NEGINF}", vr(NEGINF), vr(S(t) + r))
        # causal mask on tile w: element r is key 32w + 8(r/4) + 4lh + r%4, masked when
        # 8(r/4) + r%4 > li - 4lh
        for r in range(16):
            c = 8 * (r >> 2) + (r & 3)
            em.emit("valu", f"v_cmp_gt_i32 vcc, {c}, v{dlim}",
                    vr(dlim), ["vcc"])
            em.emit("valu", f"v_cndmask_b32 v{S(w) + r}, v{S(w) + r}, v{NEGINF}, vcc",
                    vr(S(w) + r) + vr(NEGINF) + ["vcc"], vr(S(w) + r))
        # exact row max of the diagonal block
        mx = T2 + 3
        row_max(em, list(range(w + 1)), mx)
        pair_reduce(em, mx, "v_max_f32")
        em.emit("valu", f"v_mul_f32 v{M}, {inp('scale')}, v{mx}", vr(mx), vr(M))
        # every wave has read K(b_0): refill K sub-tiles 0-2 with K(b_1)
        em.barrier()
        skip = self.L(f"nok1_{w}")
        em.raw(f"s_cmp_eq_u32 {inp('noff')}, 0")
        em.raw(f"s_cbranch_scc1 {skip}")
        for sub in range(3):
            emit_ops(em, dma_ops(KBB, sub, KL, ("ko0", "ko1")))
        em.out.append(f"{skip}:")
        # softmax of key tiles 0..2 (tile 3 runs in the first pass); tiles above the wave: P = 0
        for t in range(3):
            if t <= w:
                emit_ops(em, softmax_ops(t, LPEND))
            else:
                for ks in (2 * t, 2 * t + 1):
                    for d in range(4):
                        em.emit("valu", f"v_mov_b32 v{P(ks) + d}, 0", [], vr(P(ks) + d))
        em.emit("valu", f"v_add_f32 v{LACC}, v{LACC}, v{LPEND}", vr(LACC) + vr(LPEND), vr(LACC))
        em.emit("valu", f"v_mov_b32 v{LPEND}, 0", [], vr(LPEND))
        em.vm = []

    # ---- the pipelined pass -----------------------------------------------------------------
    def iteration(self):
        em = self.em
        loop, done = self.L("loop"), self.L("loop_end")
        em.raw(f"s_cmp_eq_u32 {inp('noff')}, 0")
        em.raw(f"s_cbranch_scc1 {done}")
        em.emit("salu", f"s_mov_b32 s{SI}, 0", [], sr(SI))
        # rotate in: KBA = K(b_1), VBA = V(b_0), VBB = V(b_1)
        em.emit("salu", f"s_mov_b64 s[{KBA}:{KBA + 1}], s[{KBB}:{KBB + 1}]", sr(KBB, 2), sr(KBA, 2))
        em.label(loop)
        # entry of b_{i+2}, existence flag, CSR column chunk reload at multiples of 64
        em.emit("salu", f"s_add_u32 s{SE}, s{SI}, 1", sr(SI), sr(SE) + ["scc"])
        em.emit("salu", f"s_cmp_lt_u32 s{SE}, {inp('noff')}", sr(SE), ["scc"])
        em.emit("salu", f"s_cselect_b32 s{SREAL}, 1, 0", ["scc"], sr(SREAL))
        if self.mode == "csr":
            norl = self.L("norl")
            em.raw(f"s_cmp_eq_u32 s{SREAL}, 0")
            em.raw(f"s_cbranch_scc1 {norl}")
            em.raw(f"s_and_b32 s{ST}, s{SE}, 63")
            em.raw(f"s_cbranch_scc1 {norl}")
            # entries e .. e+63 (clamped to the row) into colv
            em.raw(f"s_sub_u32 s{ST}, {inp('noff')}, 1")
            em.raw(f"v_add_u32 v{T2}, s{SE}, {inp('lid')}")
            em.raw(f"v_min_u32 v{T2}, s{ST}, v{T2}")
            em.raw(f"v_lshlrev_b32 v{T2}, 2, v{T2}")
            em.raw(f"s_mov_b64 s[{SCB}:{SCB + 1}], {inp('c')}")
            em.raw("s_nop 4")  # the SALU-written base and VALU-written offset before the load
            em.raw(f"global_load_dword {inp('colv')}, v{T2}, s[{SCB}:{SCB + 1}]")
            em.raw("s_waitcnt vmcnt(0)")  # also drains the tile DMAs: once per 64 entries
            em.raw("s_nop 4")  # colv before the v_readlane of the next lookup
            em.out.append(f"{norl}:")
            em.last_w = {}
            em.nops(5)
        look = kb_lookup(self.mode, SE, KBB, VBC)
        # slot 0: tile 3 of b_i, K(b_{i+1}, 3) and V(b_i, 3) refills
        self.slot(0, qk=True, sm=3, sm_sum=LT3, vmwait=(4, 8), k_refill="real", v_refill=VBA, side=[look])
        self.slot(1, qk=True, sm=0, sm_sum=LPEND, vmwait=(6, 8), k_refill="branch", v_refill=VBB)
        self.slot(2, qk=True, sm=1, sm_sum=LPEND, vmwait=8, k_refill="branch", v_refill=VBB)
        # tile 3 of b_i checked before its P·V (slot 3) and before Q·K^T overwrites S tile 3
        fb_b, ret_b = self.L("fbB"), self.L("retB")
        pre = [("valu", f"v_cmp_nge_f32 vcc, {SPEC_SUM}, v{LT3}", vr(LT3), ["vcc"])]
        self.em.wait_lgkm0()
        self.slot_check(pre, fb_b, ret_b, tail=False)
        self.slot(3, qk=True, sm=2, sm_sum=LPEND, vmwait=8, k_refill="branch", v_refill=VBB,
                  pre=[("valu", f"v_add_f32 v{LACC}, v{LACC}, v{LT3}", vr(LACC) + vr(LT3), vr(LACC)),
                       ("valu", f"v_mov_b32 v{LT3}, 0", [], vr(LT3))])
        # rotate tile bases
        em.emit("salu", f"s_mov_b64 s[{KBA}:{KBA + 1}], s[{KBB}:{KBB + 1}]", sr(KBB, 2), sr(KBA, 2))
        em.emit("salu", f"s_mov_b64 s[{VBA}:{VBA + 1}], s[{VBB}:{VBB + 1}]", sr(VBB, 2), sr(VBA, 2))
        em.emit("salu", f"s_mov_b64 s[{VBB}:{VBB + 1}], s[{VBC}:{VBC + 1}]", sr(VBC, 2), sr(VBB, 2))
        # tiles 0-2 of b_{i+1} accepted?
        fb_a, ret_a = self.L("fbA"), self.L("retA")
        em.emit("valu", f"v_cmp_nge_f32 vcc, {SPEC_SUM}, v{LPEND}", vr(LPEND), ["vcc"])
        em.raw(f"s_cbranch_vccnz {fb_a}")
        em.out.append(f"{ret_a}:")
        self.fallback_a(fb_a, ret_a)
        em.emit("valu", f"v_add_f32 v{LACC}, v{LACC}, v{LPEND}", vr(LACC) + vr(LPEND), vr(LACC))
        em.emit("valu", f"v_mov_b32 v{LPEND}, 0", [], vr(LPEND))
        em.emit("salu", f"s_add_u32 s{SI}, s{SI}, 1", sr(SI), sr(SI) + ["scc"])
        em.emit("salu", f"s_cmp_lt_u32 s{SI}, {inp('noff')}", sr(SI), ["scc"])
        em.raw(f"s_cbranch_scc1 {loop}")
        em.label(done)

    def slot_check(self, pre, fb, ret, tail):
        em = self.em
        emit_ops(em, pre)
        em.raw(f"s_cbranch_vccnz {fb}")
        em.out.append(f"{ret}:")
        self.fallback_b(fb, ret, tail)

    # ---- the last pass: P·V of b_n ----------------------------------------------------------
    def tail(self):
        em = self.em
        self.slot(0, qk=False, sm=3, sm_sum=LT3, vmwait=4, k_refill=None, v_refill=VBA)
        self.slot(1, qk=False, sm=None, sm_sum=None, vmwait=4, k_refill=None, v_refill=None)
        self.slot(2, qk=False, sm=None, sm_sum=None, vmwait=2, k_refill=None, v_refill=None)
        fb_b, ret_b = self.L("fbBt"), self.L("retBt")
        pre = [("valu", f"v_cmp_nge_f32 vcc, {SPEC_SUM}, v{LT3}", vr(LT3), ["vcc"])]
        self.slot_check(pre, fb_b, ret_b, tail=True)
        self.slot(3, qk=False, sm=None, sm_sum=None, vmwait=0, k_refill=None, v_refill=None,
                  pre=[("valu", f"v_add_f32 v{LACC}, v{LACC}, v{LT3}", vr(LACC) + vr(LT3), vr(LACC))])

    # ---- fallbacks (out of line) ------------------------------------------------------------
    def fallback_a(self, fb, ret):
        """Tiles 0-2 of b_{i+1} overflowed the speculation: exact max over all of S(b_{i+1})."""
        em = Em()
        em.out.append(f"{fb}:")
        em.nops(Em.MFMA_OTHER)
        rescale_to(em, [0, 1, 2, 3])
        em.emit("valu", f"v_mov_b32 v{LPEND}, 0", [], vr(LPEND))
        for t in range(3):
            emit_ops(em, softmax_ops(t, LPEND))
        em.nops(Em.MFMA_OTHER)
        em.raw(f"s_branch {ret}")
        self.ool += em.out

    def fallback_b(self, fb, ret, tail):
        """Tile 3 of b_i overflowed: max over it, rescale, recompute its P (and, inside the loop,
        the P of b_{i+1}'s tiles 0-1 already computed with the old max)."""
        em = Em()
        em.out.append(f"{fb}:")
        em.nops(Em.MFMA_OTHER)
        rescale_to(em, [3])
        em.emit("valu", f"v_mov_b32 v{LT3}, 0", [], vr(LT3))
        emit_ops(em, softmax_ops(3, LT3))
        if not tail:
            em.emit("valu", f"v_mov_b32 v{LPEND}, 0", [], vr(LPEND))
            for t in range(2):
                emit_ops(em, softmax_ops(t, LPEND))
        em.nops(Em.MFMA_OTHER)
        em.raw(f"s_branch {ret}")
        self.ool += em.out

    # ---- epilogue: O / l through LDS to HBM, LSE ---------------------------------------------
    def epilogue(self):
        em = self.em
        em.barrier()  # every wave is past its last LDS read of K (O is staged there)
        l, inv, e = T2 + 2, T2 + 3, T2 + 4
        em.emit("valu", f"v_mov_b32 v{l}, v{LACC}", vr(LACC), vr(l))
        pair_reduce(em, l, "v_add_f32")
        # 1 / l: v_rcp_f32 and one Newton step
        em.emit("trans", f"v_rcp_f32 v{inv}, v{l}", vr(l), vr(inv))
        em.emit("valu", f"v_fma_f32 v{e}, -v{l}, v{inv}, 1.0", vr(l) + vr(inv), vr(e))
        em.emit("valu", f"v_fma_f32 v{inv}, v{inv}, v{e}, v{inv}", vr(inv) + vr(e), vr(inv))
        # staging addresses: row li, 16-byte chunk c at (c ^ (li & 15)), half lh
        li, lh, x16, wb = 0, 1, 2, 3  # reuse S registers (dead now)
        em.emit("valu", f"v_and_b32 v{li}, 31, {inp('lid')}", [], vr(li))
        em.emit("valu", f"v_lshrrev_b32 v{lh}, 5, {inp('lid')}", [], vr(lh))
        em.emit("valu", f"v_and_b32 v{x16}, 15, v{li}", vr(li), vr(x16))
        em.emit("valu", f"v_lshlrev_b32 v{x16}, 4, v{x16}", vr(x16), vr(x16))
        em.emit("valu", f"v_lshlrev_b32 v{wb}, 8, v{li}", vr(li), vr(wb))
        em.emit("valu", f"v_lshl_add_u32 v{wb}, v{lh}, 3, v{wb}", vr(lh) + vr(wb), vr(wb))
        em.emit("valu", f"v_add_u32 v{wb}, s{STG}, v{wb}", vr(wb), vr(wb))
        ov = list(range(8, 12))
        pk = [12, 13]
        addr = 14
        for u in range(4):
            for g in range(4):
                for k in range(4):
                    em.emit("valu", f"v_accvgpr_read_b32 v{ov[k]}, a{16 * u + 4 * g + k}", ar(16 * u + 4 * g + k), vr(ov[k]))
                for k in range(4):
                    em.emit("valu", f"v_mul_f32 v{ov[k]}, v{ov[k]}, v{inv}", vr(ov[k]) + vr(inv), vr(ov[k]))
                cvt = "v_cvt_pk_bf16_f32" if self.bf16 else "v_cvt_pk_f16_f32"
                em.emit("valu", f"{cvt} v{pk[0]}, v{ov[0]}, v{ov[1]}", vr(ov[0]) + vr(ov[1]), vr(pk[0]))
                em.emit("valu", f"{cvt} v{pk[1]}, v{ov[2]}, v{ov[3]}", vr(ov[2]) + vr(ov[3]), vr(pk[1]))
                c = 4 * u + g
                em.emit("valu", f"v_xor_b32 v{addr}, {16 * c}, v{x16}", vr(x16), vr(addr))
                em.emit("valu", f"v_add_u32 v{addr}, v{addr}, v{wb}", vr(addr) + vr(wb), vr(addr))
                em.emit("ds", f"ds_write_b64 v{addr}, v[{pk[0]}:{pk[1]}]", vr(addr) + vr(pk[0], 2), [])
        em.raw("s_waitcnt lgkmcnt(0)")
        em.lgkm = []
        # whole rows back: row 4i + L/16 (i < 8), chunk L & 15 at (L & 15) ^ (row & 15)
        rb, y16, oo = 20, 21, 22
        em.emit("valu", f"v_lshrrev_b32 v{rb}, 4, {inp('lid')}", [], vr(rb))           # L / 16
        em.emit("valu", f"v_and_b32 v{y16}, 15, {inp('lid')}", [], vr(y16))            # L & 15
        em.emit("valu", f"v_lshlrev_b32 v{oo}, 4, v{y16}", vr(y16), vr(oo))
        em.emit("valu", f"v_lshl_add_u32 v{oo}, v{rb}, 8, v{oo}", vr(rb) + vr(oo), vr(oo))  # global offset
        em.emit("valu", f"v_xor_b32 v{y16}, v{y16}, v{rb}", vr(y16) + vr(rb), vr(y16))
        em.emit("valu", f"v_lshlrev_b32 v{y16}, 4, v{y16}", vr(y16), vr(y16))
        em.emit("valu", f"v_lshlrev_b32 v{rb}, 8, v{rb}", vr(rb), vr(rb))
        em.emit("valu", f"v_add_u32 v{rb}, s{STG}, v{rb}", vr(rb), vr(rb))
        vals = [24 + 4 * i for i in range(8)]
        for i in range(4):
            a = 56 + i
            em.emit("valu", f"v_xor_b32 v{a}, {64 * i}, v{y16}", vr(y16), vr(a))
            em.emit("valu", f"v_add_u32 v{a}, v{a}, v{rb}", vr(a) + vr(rb), vr(a))
            em.emit("ds", f"ds_read_b128 v[{vals[i]}:{vals[i] + 3}], v{a} offset:{1024 * i}", vr(a), vr(vals[i], 4))
            em.emit("ds", f"ds_read_b128 v[{vals[i + 4]}:{vals[i + 4] + 3}], v{a} offset:{1024 * i + 4096}", vr(a), vr(vals[i + 4], 4))
        em.emit("salu", f"s_mov_b64 s[{SX}:{SX + 1}], {inp('o')}", [], sr(SX, 2))
        em.emit("salu", f"s_add_u32 s{SP}, s{SX}, 4096", sr(SX), sr(SP) + ["scc"])
        em.emit("salu", f"s_addc_u32 s{SP + 1}, s{SX + 1}, 0", sr(SX + 1) + ["scc"], sr(SP + 1) + ["scc"])
        for i in range(8):
            base = SX if i < 4 else SP
            em.emit("vmem", f"global_store_dwordx4 v{oo}, v[{vals[i]}:{vals[i] + 3}], s[{base}:{base + 1}] offset:{1024 * (i % 4)} nt",
                    vr(oo) + vr(vals[i], 4) + sr(base, 2), [])
        # LSE = (m + log2 l) ln 2 for lanes 0-31 (one per row)
        nolse = self.L("nolse")
        em.raw(f"s_cmp_eq_u32 {inp('haslse')}, 0")
        em.raw(f"s_cbranch_scc1 {nolse}")
        lg, lo = 60, 61
        em.emit("trans", f"v_log_f32 v{lg}, v{l}", vr(l), vr(lg))
        em.emit("valu", f"v_add_f32 v{lg}, v{M}, v{lg}", vr(M) + vr(lg), vr(lg))
        em.emit("valu", f"v_mul_f32 v{lg}, 0x3f317218, v{lg}", vr(lg), vr(lg))
        em.emit("valu", f"v_lshlrev_b32 v{lo}, 2, v{li}", vr(li), vr(lo))
        em.emit("salu", f"s_mov_b64 s[{SX}:{SX + 1}], {inp('l')}", [], sr(SX, 2))
        em.raw("s_mov_b32 exec_hi, 0")
        em.raw("s_nop 1")
        em.emit("vmem", f"global_store_dword v{lo}, v{lg}, s[{SX}:{SX + 1}]", vr(lo) + vr(lg) + sr(SX, 2), [])
        em.raw("s_mov_b64 exec, -1")
        em.raw("s_nop 1")
        em.out.append(f"{nolse}:")
        em.raw("s_waitcnt vmcnt(0)")

    def build(self):
        self.prologue()
        self.iteration()
        self.tail()
        self.epilogue()
        done = self.L("end")
        self.em.raw(f"s_branch {done}")
        return self.em.out + self.ool + [f"{done}:"]


# ------------------------------------------------------------------------------------------
# output
# ------------------------------------------------------------------------------------------

HEADER = """// Generated by gen_bsa_pipe.py; do not edit. Inline assembly of bsa_fwd_pipe_kernel's work
// item (one string per row kind and input type). Operands: see the asm statement in bsa_fwd.hip.
"""


def c_string(lines):
    out = []
    for ln in lines:
        esc = ln.replace("\\", "\\\\").replace('"', '\\"')
        out.append(f'  "{esc}\\n\\t"')
    return "\n".join(out)


def generate():
    parts = [HEADER]
    for mode, bf16, name in (("csr", False, "USAGI_PIPE_ASM_CSR_F16"), ("window", False, "USAGI_PIPE_ASM_WINDOW_F16"),
                             ("csr", True, "USAGI_PIPE_ASM_CSR_BF16"), ("window", True, "USAGI_PIPE_ASM_WINDOW_BF16")):
        k = Kernel(mode, bf16)
        lines = k.build()
        parts.append(f"#define {name} \\\n" + c_string(lines).replace("\n", " \\\n") + "\n")
    parts.append(f"#define USAGI_PIPE_SGPR_LO {SGPR_LO}\n#define USAGI_PIPE_SGPR_HI {SGPR_HI}\n"
                 f"#define USAGI_PIPE_LAST_VGPR {LAST_V}\n#define USAGI_PIPE_AGPRS {N_AGPR}\n")
    return "\n".join(parts)


OUT_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "bsa_pipe_asm.inc")


def write(path: str = OUT_PATH) -> str:
    """Write the include file (only if its contents change) and return its path."""
    text = generate()
    cur = open(path).read() if os.path.exists(path) else None
    if cur != text:
        tmp = path + ".tmp"
        with open(tmp, "w") as f:
            f.write(text)
        os.replace(tmp, path)
    return path


def main(argv):
    out = OUT_PATH
    text = generate()
    if len(argv) > 1 and argv[1] == "--check":
        cur = open(out).read() if os.path.exists(out) else ""
        sys.exit(0 if cur == text else 1)
    with open(out, "w") as f:
        f.write(text)


if __name__ == "__main__":
    main(sys.argv)
