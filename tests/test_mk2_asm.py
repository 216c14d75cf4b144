"""The persistent verify kernel's inline-asm weight ring is safe as compiled
(CPU: builds csrc/mk2.hip to AMD assembly with hipcc, no GPU needed).

The ring's loads and waits are inline asm the compiler cannot see, so two
invariants hold only by construction (tests/asm_slots.py): nothing touches a
slot register while its load may be in flight, and each SLOTWAIT's vmcnt
really covers its slot on every path.  The checker itself is shown to catch
both kinds of violation, seeded into the real listing and into a small
hand-written one."""
import os
import subprocess

import pytest

import asm_slots

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "s2pro-native_amd")
HIPCC = "/opt/rocm/bin/hipcc"


@pytest.fixture(scope="module")
def mk2_asm(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc is not installed")
    out = tmp_path_factory.mktemp("asm") / "mk2.s"
    # the flags of the library build of mk2.hip (s2pro-native_amd/Makefile)
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fno-gpu-flush-denormals-to-zero",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(PKG, "csrc"),
           "-mllvm", "-amdgpu-mfma-vgpr-form=1", "--cuda-device-only", "-S",
           os.path.join(PKG, "csrc", "mk2.hip"), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    return out.read_text()


def test_library_flags_match_the_check():
    """The check compiles mk2.hip with the Makefile's flags for it."""
    mk = open(os.path.join(PKG, "Makefile")).read()
    assert "-mllvm -amdgpu-mfma-vgpr-form=1" in mk
    assert "-O3" in mk and "--offload-arch=$(ARCH)" in mk


def test_ring_slots_clean(mk2_asm):
    bad, stats = asm_slots.check(mk2_asm)
    print(stats)
    assert stats["slot_loads"] > 0 and stats["slot_waits"] > 0
    assert not bad, "\n".join(bad[:20])


def test_checker_catches_a_short_wait(mk2_asm):
    """One SLOTWAIT loosened by one count no longer covers its slot."""
    i = mk2_asm.index("SLOTWAIT")
    j = mk2_asm.rfind("vmcnt(", 0, i)
    n = int(mk2_asm[j + 6:mk2_asm.index(")", j)])
    seeded = mk2_asm[:j] + f"vmcnt({n + 1})" + mk2_asm[mk2_asm.index(")", j) + 1:]
    bad, _ = asm_slots.check(seeded)
    assert any("does not cover" in b for b in bad), bad[:5]


def test_checker_catches_an_early_read(mk2_asm):
    """A read of a slot register right after its load is reported."""
    k = mk2_asm.index("SLOTLOAD")
    line = mk2_asm[mk2_asm.rfind("\n", 0, k) + 1:k]
    dest = line.split()[1].rstrip(",")            # e.g. a[8:11]
    reg = dest if "[" not in dest else dest[0] + dest[2:dest.index(":")]
    e = mk2_asm.index("\n", mk2_asm.index(";;#ASMEND", k))
    seeded = mk2_asm[:e + 1] + f"\tv_accvgpr_read_b32 v0, {reg}\n" + mk2_asm[e + 1:]
    bad, _ = asm_slots.check(seeded)
    assert any("touches in-flight" in b and reg[1:] in b for b in bad), bad[:5]


SMALL = """
k:
\t;;#ASMSTART
\t; CPATH_BEGIN
\t;;#ASMEND
\t;;#ASMSTART
\tglobal_load_dwordx4 a[0:3], v1, s[2:3] nt ; SLOTLOAD
\t;;#ASMEND
\tglobal_load_dword v9, v1, s[2:3]
\ts_cbranch_scc1 .LBB0_2
\tglobal_load_dword v10, v1, s[2:3]
.LBB0_2:
\ts_waitcnt vmcnt(0)
\t;;#ASMSTART
\ts_waitcnt vmcnt({n}) ; SLOTWAIT a[0:3] a[4:5]
\t;;#ASMEND
\tv_accvgpr_read_b32 v2, a1
\ts_endpgm
"""


def test_checker_on_a_small_listing():
    """vmcnt(1) covers the slot on both paths (one load issued after it on
    the short path); vmcnt(2) does not (the path that skips the second load);
    a read before the wait is reported."""
    ok = SMALL.replace("\ts_waitcnt vmcnt(0)\n", "")
    assert asm_slots.check(ok.format(n=1))[0] == []
    bad, _ = asm_slots.check(ok.format(n=2))
    assert len(bad) == 1 and "does not cover" in bad[0]
    early = ok.replace("\ts_cbranch_scc1", "\tv_mov_b32 v3, a2\n\ts_cbranch_scc1")
    bad, _ = asm_slots.check(early.format(n=1))
    assert len(bad) == 1 and "touches in-flight" in bad[0]
    # a compiler wait for everything retires the slot before the asm wait
    assert asm_slots.check(SMALL.format(n=7))[0] == []
