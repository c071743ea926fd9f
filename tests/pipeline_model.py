"""Host restatement of the INT8 tile GEMM's LDS pipeline, for CPU checks of its
addresses and wait budgets.

Test infrastructure. `gemm_programs` lists, per wave of one workgroup, the operations of
gemm_tile (krea2-hrx_amd/csrc/k2w8_gemm.hip) that touch LDS or order it: transfers into a
stage (global_load_lds), `s_waitcnt vmcnt(n)`, `s_waitcnt lgkmcnt(0)`, barriers, the
fragment reads of a K step, and the epilogue's staging writes and reads. `check` then
proves, for every interleaving the barriers allow, that each read sees the transfers it
needs completed and no other transfer into the same bytes in flight, and that no
transfer or read overlaps an epilogue write. It relies on one property of the hardware:
a wave's vector-memory loads (global_load_lds included) complete in issue order, so
`vmcnt(n)` leaves at most the n newest outstanding. `transfer_map` restates the
addresses: which global row and 16-byte chunk each lane's transfer brings to which LDS
byte, against the swizzle the fragment reads assume.

The skinny kernel (k2w8_skinny.hip, one ring per wave and no barriers in the K loop) has
its own restatement in `skinny_program`.
"""

from __future__ import annotations

from dataclasses import dataclass

PLAIN, RESID, SWIGLU, BIAS, ACC = 0, 1, 2, 3, 4


@dataclass(frozen=True)
class Tile:
    bm: int
    bn: int
    wm: int
    wn: int
    bk: int
    stages: int
    epi: int
    kg: int = 1

    @property
    def waves(self):
        return self.wm * self.wn * self.kg

    @property
    def a_ins(self):
        return self.bm * self.bk // 1024 // self.waves

    @property
    def b_ins(self):
        return self.bn * self.bk // 1024 // self.waves

    @property
    def split_roles(self):
        return self.waves == 8

    @property
    def producers(self):
        return self.waves // 2 if self.split_roles else self.waves

    @property
    def per(self):  # virtual waves per producer
        return 2 if self.split_roles else 1

    @property
    def budget(self):  # a producer's transfers per stage
        return self.per * (self.a_ins + self.b_ins)

    @property
    def stage_bytes(self):
        return (self.bm + self.bn) * self.bk

    @property
    def fm(self):
        return self.bm // self.wm // 32

    @property
    def fn(self):
        return self.bn // self.wn // 32

    @property
    def ops_bytes(self):  # EpiOperands<BM, BN>::kBytes
        return self.bn * 8 + self.bm * 4

    @property
    def region(self):  # gemm_tile's kRegion
        cols = 16 * self.fn if self.epi == SWIGLU else 32 * self.fn
        return 32 * (cols * (4 if self.epi == ACC else 2) + 16)

    @property
    def overflow(self):  # EpiStaging<...>::kOverflow (sized for 16-bit outputs)
        cw = self.wm * self.wn
        region = 32 * (32 * self.fn * 2 + 16)
        per_stage = min(self.stage_bytes // region, cw)
        return (cw - per_stage) * region if self.kg == 1 else 0

    @property
    def lds_bytes(self):  # TileConfig<...>::kLds, the launch's dynamic LDS
        return self.stages * self.stage_bytes + self.ops_bytes + self.overflow

    def waits(self):
        """(prologue, loop) vmcnt budgets of a producer, as gemm_tile sets them."""
        return (self.stages - 1) * self.budget, (self.stages - 2) * self.budget


def gemm_programs(t: Tile, kt_count: int, prologue_wait=None, loop_wait=None):
    """Per-wave operation lists of one workgroup running `kt_count` K steps."""
    pro, loop = t.waits()
    pro = pro if prologue_wait is None else prologue_wait
    loop = loop if loop_wait is None else loop_wait
    S, stage = t.stages, t.stage_bytes

    def st(s):
        return (s * stage, (s + 1) * stage)

    ops = (S * stage, S * stage + t.ops_bytes)
    ns = t.bk // 32 // t.kg
    cw_count = t.wm * t.wn
    progs = []
    for w in range(t.waves):
        p, producer = [], w < t.producers
        if w == 0 and t.epi != ACC:
            p.append(("dma", "E", ops))
        for s in range(min(S, kt_count)):
            if producer:
                p += [("dma", s, st(s))] * t.budget
        if kt_count < S:
            p.append(("wait", 0))
        elif producer:
            p.append(("wait", pro))
        p.append(("bar",))
        p.append(("read", 0, st(0)))
        for k in range(kt_count):
            if ns > 1:
                p.append(("read", k, st(k % S)))  # the step's other slices
            p.append(("lgkm0",))  # the last slice drains its LDS reads
            if k + 1 < kt_count:
                p.append(("wait", loop if k + S - 1 < kt_count else 0))
                p.append(("bar",))
                if k + S < kt_count and producer:
                    p += [("dma", k + S, st((k + S) % S))] * t.budget
                p.append(("read", k + 1, st((k + 1) % S)))
        p += epilogue_ops(t, w, kt_count, cw_count, ops)
        progs.append(p)
    return progs


def epilogue_ops(t: Tile, w: int, kt_count: int, cw_count: int, ops):
    """The epilogue's LDS operations of wave w (the four forms of gemm_tile)."""
    S, stage, region = t.stages, t.stage_bytes, t.region
    uses_ops = t.epi != ACC
    out = []
    if t.kg > 1:
        kg, cw = divmod(w, cw_count)
        part = t.fm * t.fn * 64 * 64
        group_sums = cw_count * part
        assert region * cw_count + (t.kg - 1) * group_sums <= S * stage
        out += [("lgkm0",), ("bar",)]
        if kg > 0:
            lo = region * cw_count + (kg - 1) * group_sums + cw * part
            out.append(("write", ("sums", kg, cw), (lo, lo + part)))
        out.append(("bar",))
        if kg > 0:
            return out
        for k in range(1, t.kg):
            lo = region * cw_count + (k - 1) * group_sums + cw * part
            out.append(("read", ("sums", k, cw), (lo, lo + part)))
        mine = (cw * region, (cw + 1) * region)
    else:
        per = min(stage // region, t.waves)
        if (t.waves - per) * region <= t.overflow:
            free = (kt_count - 2) % S if kt_count >= 2 else 1
            if w < per:
                lo = free * stage + w * region
            else:
                lo = S * stage + t.ops_bytes + (w - per) * region
            mine = (lo, lo + region)
        elif region * t.waves <= S * stage:
            out += [("lgkm0",), ("bar",)]
            mine = (w * region, (w + 1) * region)
        else:
            return out + ([("read", "E", ops)] if uses_ops else [])  # direct stores
    out.append(("write", ("epi", w), mine))
    out.append(("read", ("epi", w), mine))
    if uses_ops:
        out.append(("read", "E", ops))
    return out


def _overlap(a, b):
    return a[0] < b[1] and b[0] < a[1]


def check(progs, lds_bytes=None):
    """Violations (strings) of the LDS ordering rules over every interleaving the
    barriers allow; [] when the pipeline is race-free."""
    bad = []
    bars = {sum(op[0] == "bar" for op in p) for p in progs}
    if len(bars) != 1:
        return [f"waves reach different numbers of barriers: {sorted(bars)}"]
    dmas, reads, writes = [], [], []
    for w, p in enumerate(progs):
        epoch, mine = 0, []
        for pos, op in enumerate(p):
            kind = op[0]
            if kind == "bar":
                epoch += 1
            elif kind == "dma":
                d = dict(wave=w, group=op[1], region=op[2], epoch=epoch, pos=pos, done=None)
                dmas.append(d)
                mine.append(d)
            elif kind == "wait":
                pending = [d for d in mine if d["done"] is None]
                for d in pending[:max(0, len(pending) - op[1])]:
                    d["done"] = (epoch, pos)
            elif kind in ("read", "write"):
                # the LDS access completes at the next lgkmcnt(0) (reads) before a barrier
                end = None
                e2 = epoch
                for pos2 in range(pos + 1, len(p)):
                    if p[pos2][0] == "bar":
                        e2 += 1
                    if p[pos2][0] == "lgkm0":
                        end = (e2, pos2)
                        break
                rec = dict(wave=w, tag=op[1], region=op[2], epoch=epoch, pos=pos, end=end)
                (reads if kind == "read" else writes).append(rec)
        for d in mine:
            if d["done"] is None:
                bad.append(f"wave {w}: transfer of group {d['group']} never waited for")
    if lds_bytes is not None:
        for x in dmas + reads + writes:
            if not (0 <= x["region"][0] < x["region"][1] <= lds_bytes):
                bad.append(f"LDS range {x['region']} outside the launch's {lds_bytes} bytes")

    def visible(d, w, epoch, pos):
        if d["done"] is None:
            return False
        if d["wave"] == w:
            return d["done"][1] < pos
        return d["done"][0] < epoch

    def read_done_before(r, w, epoch, pos):
        # r (an LDS read) has completed before (w, epoch, pos): its lgkmcnt(0) came in an
        # earlier epoch, or earlier in the same wave
        if r["end"] is None:
            return False
        if r["wave"] == w:
            return r["end"][1] < pos
        return r["end"][0] < epoch

    for r in reads:
        w, e, pos, tag = r["wave"], r["epoch"], r["pos"], r["tag"]
        if isinstance(tag, int) or tag == "E":
            need = [d for d in dmas if d["group"] == tag and _overlap(d["region"], r["region"])]
            if not need:
                bad.append(f"wave {w}: read of group {tag} that no transfer writes")
            for d in need:
                if not visible(d, w, e, pos):
                    bad.append(f"wave {w} reads group {tag} before wave {d['wave']}'s transfer is done")
                    break
            for d in dmas:
                if d["group"] == tag or not _overlap(d["region"], r["region"]):
                    continue
                older = isinstance(d["group"], int) and isinstance(tag, int) and d["group"] < tag
                if older and visible(d, w, e, pos):
                    continue  # overwritten by `tag`'s transfer, which is complete
                later = r["end"] is not None and (
                    (d["wave"] == w and d["pos"] > r["end"][1]) or d["epoch"] > r["end"][0])
                if not later:
                    bad.append(f"wave {w}'s read of group {tag} may see wave {d['wave']}'s transfer of "
                               f"group {d['group']}")
                    break
        else:  # an LDS read of staged epilogue data (or K-group sums)
            src = [x for x in writes if x["tag"] == tag]
            if not src:
                bad.append(f"wave {w} reads {tag}, which nobody writes")
            for x in src:
                if not ((x["wave"] == w and x["pos"] < pos) or x["epoch"] < e):
                    bad.append(f"wave {w} reads {tag} before wave {x['wave']} writes it")
            for d in dmas:
                if _overlap(d["region"], r["region"]) and not visible(d, w, e, pos):
                    bad.append(f"wave {w}'s read of {tag} may see wave {d['wave']}'s transfer of "
                               f"group {d['group']}")
                    break
    for x in writes:
        w, e, pos = x["wave"], x["epoch"], x["pos"]
        for d in dmas:
            if _overlap(d["region"], x["region"]) and not visible(d, w, e, pos):
                bad.append(f"wave {w}'s write of {x['tag']} overlaps wave {d['wave']}'s transfer of "
                           f"group {d['group']} in flight")
                break
        for r in reads:
            if r["wave"] != w and r["tag"] != x["tag"] and _overlap(r["region"], x["region"]) and \
                    not read_done_before(r, w, e, pos):
                bad.append(f"wave {w}'s write of {x['tag']} may overwrite what wave {r['wave']} still "
                           f"reads ({r['tag']})")
                break
        for y in writes:
            if y is not x and y["wave"] != w and _overlap(y["region"], x["region"]):
                bad.append(f"waves {w} and {y['wave']} write overlapping LDS ({x['tag']}, {y['tag']})")
                break
    return bad


def swz_key(bk: int, row: int) -> int:
    return (row >> 1) & (bk // 16 - 1)


def transfer_map(t: Tile):
    """Every 16-byte LDS chunk of one stage that the producers' transfers write, as
    (LDS offset within the stage) -> (operand, row in the tile, logical K chunk), by the
    kernel's formulas for the transfer instruction, lane and swizzle; and every fragment
    read as (wave, lane, slice, operand block) -> LDS offset."""
    rows_per_kb, cpr = 1024 // t.bk, t.bk // 16
    writes = {}
    for wave in range(t.producers):
        for j in range(t.per):
            v = wave + j * t.producers  # virtual wave
            for operand, ins, base in (("a", t.a_ins, 0), ("b", t.b_ins, t.bm * t.bk)):
                lds_wave = base + v * ins * 1024
                for i in range(ins):
                    m0 = lds_wave + i * 1024  # the instruction's LDS base (M0)
                    for lane in range(64):
                        row = (v * ins + i) * rows_per_kb + lane // cpr
                        logical = (lane % cpr) ^ swz_key(t.bk, row)
                        off = m0 + 16 * lane
                        assert off not in writes, ("two transfers write", off)
                        writes[off] = (operand, row, logical)
    reads = {}
    cw_count = t.wm * t.wn
    ns = t.bk // 32 // t.kg
    for wave in range(t.waves):
        kg, cw = divmod(wave, cw_count)
        wm, wn = divmod(cw, t.wn)
        for lane in range(64):
            fr, kh = lane & 31, lane >> 5
            rsw = swz_key(t.bk, fr)
            for s in range(ns):
                chunk = ((2 * (kg * ns + s) + kh) ^ rsw) << 4
                for i in range(t.fm):
                    row = wm * (t.bm // t.wm) + i * 32 + fr
                    reads[(wave, lane, s, "a", i)] = ("a", row, 2 * (kg * ns + s) + kh,
                                                      row * t.bk + chunk)
                for j in range(t.fn):
                    row = wn * (t.bn // t.wn) + j * 32 + fr
                    reads[(wave, lane, s, "b", j)] = ("b", row, 2 * (kg * ns + s) + kh,
                                                      t.bm * t.bk + row * t.bk + chunk)
    return writes, reads


def skinny_program(p: int, i: int, count: int, wait_of=None):
    """One wave of the skinny kernel's K loop: `count` 128-byte steps through a ring of
    p slots, `i` transfers per step. `wait_of(newer)` is the vmcnt the kernel waits for
    with `newer` younger steps in flight (default: newer * i, as wait_steps sets)."""
    wait_of = wait_of or (lambda newer: newer * i)
    slot = lambda s: (s % p, s % p + 1)  # noqa: E731
    prog = []
    for s in range(min(p, count)):
        prog += [("dma", s, slot(s))] * i
    for st in range(count):
        prog.append(("wait", wait_of(min(count - 1 - st, p - 1))))
        prog.append(("read", st, slot(st)))
        prog.append(("lgkm0",))
        if st + p < count:
            prog += [("dma", st + p, slot(st + p))] * i
    prog += [("lgkm0",), ("bar",)]  # __syncthreads before the partial sums reuse the ring
    return [prog]
