"""Invariants of the built device code, checked on the CPU from the gfx950 code objects
in libkrea2_w8a8.so and a host restatement of the tile GEMM's LDS pipeline.

The GEMM and few-token kernels move operands global -> LDS with global_load_lds
instructions issued through inline asm, and wait for them with hand-counted
`s_waitcnt vmcnt(n)` (the compiler's own wait counting does not see asm). What makes
those counts right:
- a wave's vector-memory loads complete in issue order, so `vmcnt(n)` leaves only the
  n newest outstanding; any other load or store the compiler adds only makes a wait
  stricter, never looser;
- the budgets: before reading stage k + 1, a producer has at most the transfers of the
  stages after it in flight ((STAGES - 2) x its transfers per stage), and before the
  first read (STAGES - 1) x;
- every wave drains its LDS reads (lgkmcnt(0)) before the barrier after which a
  transfer may refill what it read.
The tests below hold each of these: the waits in the machine code against the budget
formula, the formula's schedule against every interleaving the barriers allow
(pipeline_model.check), the drain before each barrier by data flow over the kernel's
control-flow graph, and the transfer and fragment-read addresses against each other.
Kernels that transfer this way also must not use scratch memory: it is a second kind
of vector-memory traffic in the pipeline, and a spill there is a sign of register
pressure the tile was not designed for.
"""

import collections
import os
import re
import shutil
import subprocess

import pytest

import codeobj
import isa_cfg
import pipeline_model as pm

pytestmark = pytest.mark.skipif(shutil.which("/opt/rocm/llvm/bin/llvm-objdump") is None,
                                reason="needs the ROCm LLVM tools")

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module", autouse=True)
def built():
    if not os.path.exists(codeobj.LIB):
        subprocess.run(["make", "-s", "-C", os.path.dirname(codeobj.LIB)], check=True)


def _template_ints(name, kernel):
    seg = name[name.index(kernel + "I") + len(kernel) + 1:]
    seg = seg[:seg.index("EEv")]
    return [int(x) for x in re.findall(r"Li(\d+)E", seg)]


def _kernels(kernel):
    out = []
    for k in codeobj.kernels():
        if f"{len(kernel)}{kernel}I" in k[".name"]:
            lines = codeobj.disassembly(k[".image"])[k[".name"]]
            out.append((k, _template_ints(k[".name"], kernel), isa_cfg.build(lines)))
    return out


def _gemm_tiles():
    tiles = []
    for k, args, blocks in _kernels("gemm_kernel"):
        bm, bn, wm, wn, bk, stages, epi, kg = args
        tiles.append((k[".name"], pm.Tile(bm, bn, wm, wn, bk, stages, epi, kg), blocks))
    # the backward-K forms (one K group): the same LDS schedule, other global offsets
    for k, args, blocks in _kernels("gemm_kernel_backward"):
        bm, bn, wm, wn, bk, stages, epi = args
        tiles.append((k[".name"], pm.Tile(bm, bn, wm, wn, bk, stages, epi), blocks))
    assert len(tiles) >= 48, "the tile kernels the build instantiates"
    return tiles


def _uses_transfers(k):
    lines = codeobj.disassembly(k[".image"])[k[".name"]]
    return any(line.startswith("global_load_lds") for line in lines)


def test_kernels_that_transfer_to_lds_use_no_scratch():
    checked = 0
    for k in codeobj.kernels():
        assert k[".uses_dynamic_stack"] is False, k[".name"]
        if not _uses_transfers(k):
            continue
        checked += 1
        lines = codeobj.disassembly(k[".image"])[k[".name"]]
        assert k[".private_segment_fixed_size"] == 0, k[".name"]
        # (SGPR spills go to VGPR lanes, not memory: allowed)
        assert k[".vgpr_spill_count"] == 0, k[".name"]
        assert not any(line.startswith("scratch_") for line in lines), k[".name"]
    assert checked >= 100  # tile GEMMs, few-token kernels, fused, attention


def test_gemm_waits_in_the_machine_code_are_the_budget():
    for name, t, blocks in _gemm_tiles():
        got = set(isa_cfg.pipeline_waits(blocks))
        pro, loop = t.waits()
        assert got == {0, pro, loop}, (name, sorted(got), (pro, loop))


@pytest.mark.parametrize("kt_extra", [0, 1, 2, 3, 9])
def test_gemm_pipeline_is_race_free_with_the_machine_codes_waits(kt_extra):
    # The waits read out of each kernel's code (the largest is the prologue's, the next
    # the loop's), run through every K-step count from one step to past the ring.
    for name, t, blocks in _gemm_tiles():
        waits = sorted(set(isa_cfg.pipeline_waits(blocks)), reverse=True)
        pro, loop = waits[0], (waits[1] if len(waits) > 1 else 0)
        assert t.lds_bytes <= 160 * 1024, name
        for kt in range(1, t.stages + 1) if kt_extra == 0 else [t.stages + kt_extra]:
            bad = pm.check(pm.gemm_programs(t, kt, pro, loop), t.lds_bytes)
            assert bad == [], (name, kt, bad[:3])


@pytest.mark.parametrize("tile", [pm.Tile(256, 192, 4, 2, 128, 2, pm.PLAIN),
                                  pm.Tile(128, 64, 4, 2, 128, 3, pm.RESID),
                                  pm.Tile(64, 64, 2, 2, 128, 4, pm.PLAIN, 2),
                                  pm.Tile(256, 128, 4, 2, 128, 3, pm.SWIGLU)])
def test_the_model_catches_a_wrong_budget(tile):
    pro, loop = tile.waits()
    assert pm.check(pm.gemm_programs(tile, 12), tile.lds_bytes) == []
    # one stage's transfers too many left in flight, at either wait
    assert pm.check(pm.gemm_programs(tile, 12, loop_wait=loop + tile.budget), tile.lds_bytes)
    assert pm.check(pm.gemm_programs(tile, 12, prologue_wait=pro + tile.budget), tile.lds_bytes)
    # one transfer too many is enough
    assert pm.check(pm.gemm_programs(tile, 12, loop_wait=loop + 1), tile.lds_bytes)
    # reads not drained before the barrier that lets the refill go
    progs = [[op for op in p if op[0] != "lgkm0"] for p in pm.gemm_programs(tile, 12)]
    assert pm.check(progs, tile.lds_bytes)


def test_no_barrier_follows_an_lds_read_that_was_not_waited_for():
    checked = 0
    for k in codeobj.kernels():
        if not _uses_transfers(k):
            continue
        blocks = isa_cfg.build(codeobj.disassembly(k[".image"])[k[".name"]])
        assert isa_cfg.barriers_after_unfinished_lds_reads(blocks) == [], k[".name"]
        checked += 1
    assert checked >= 100


def test_transfers_and_fragment_reads_agree_on_every_address():
    for name, t, _ in _gemm_tiles():
        if t.epi != pm.PLAIN:
            continue  # the addresses do not depend on the epilogue
        writes, reads = pm.transfer_map(t)
        # the producers' transfers write every 16-byte chunk of a stage exactly once
        assert sorted(writes) == list(range(0, t.stage_bytes, 16)), name
        for off, (operand, row, logical) in writes.items():
            base = 0 if operand == "a" else t.bm * t.bk
            assert row < (t.bm if operand == "a" else t.bn)
            assert off == base + row * t.bk + ((logical ^ pm.swz_key(t.bk, row)) << 4), (name, off)
        # every fragment read finds the row and K chunk it multiplies
        seen = collections.defaultdict(set)
        for key, (operand, row, logical, off) in reads.items():
            assert writes[off] == (operand, row, logical), (name, key)
            seen[operand].add((row, logical))
        assert len(seen["a"]) == t.bm * t.bk // 16 and len(seen["b"]) == t.bn * t.bk // 16, name


def test_few_token_kernel_waits_and_ring():
    kernels = _kernels("stream_kernel")
    assert len(kernels) >= 40
    for k, (rb, tb, ar, waves, p, epi), blocks in kernels:
        ins = rb // 8 + tb * ar // 8  # transfers per step (wait_steps's I)
        got = set(isa_cfg.pipeline_waits(blocks))
        assert got <= {n * ins for n in range(p)} and (p - 1) * ins in got, (k[".name"], sorted(got))
        for count in range(0, p + 4):
            assert pm.check(pm.skinny_program(p, ins, count)) == [], (k[".name"], count)
    # and a ring that waits one step short is caught
    assert pm.check(pm.skinny_program(4, 3, 9, wait_of=lambda newer: (newer + 1) * 3))
