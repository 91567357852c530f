"""The build check on m0 (candle-3d_amd/check_m0.py): the inline-assembly
direct-to-LDS loads set m0 themselves, so the build must fail when the
compiler keeps anything of its own in m0 in the same translation unit.
Checked here on small assembly texts (clean pairs pass; a compiler-set m0,
an asm block that is not the pair, and an implicit m0 user each fail), on
the device assembly the build wrote, and that every source calling the
loads is in the Makefile's checked list."""
import os
import re
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "candle-3d_amd")
sys.path.insert(0, PKG)
import check_m0  # noqa: E402

PAIR = """\t;;#ASMSTART
\ts_mov_b32 m0, s8
\tbuffer_load_dwordx4 v146, s[0:3], s9 offen lds
\t;;#ASMEND
"""


def _run(tmp_path, body):
    p = tmp_path / "k.s"
    p.write_text("_Z6kernelv:                              ; @_Z6kernelv\n" + body + "\ts_endpgm\n")
    return check_m0.check(str(p))


def test_clean_pairs_pass(tmp_path):
    bad, nfunc, pairs = _run(tmp_path, PAIR + "\tv_mov_b32 v0, 0\n" + PAIR.replace("dwordx4", "dword"))
    assert bad == [] and nfunc == 1 and pairs == 2


@pytest.mark.parametrize("body,what", [
    ("\ts_mov_b32 m0, s12\n" + PAIR + "\ts_add_i32 s1, m0, 4\n", "compiler-generated use of m0"),
    ("\t;;#ASMSTART\n\ts_mov_b32 m0, s8\n\ts_nop 0\n\tbuffer_load_dword v1, s[0:3], 0 offen lds\n\t;;#ASMEND\n",
     "not the s_mov_b32 m0"),
    (PAIR + "\ts_sendmsg sendmsg(MSG_DEALLOC_VGPRS)\n", "implicitly"),
    (PAIR + "\tbuffer_load_dwordx4 v1, s[0:3], 0 offen lds\n", "implicitly"),
    (PAIR + "\tv_movrels_b32 v0, v1\n", "implicitly"),
])
def test_violations_fail(tmp_path, body, what):
    bad, _, _ = _run(tmp_path, body)
    assert bad and what in bad[0]


def test_every_lds_load_caller_is_checked():
    mk = open(os.path.join(PKG, "Makefile")).read()
    checked = set(re.search(r"^M0_SRCS\s*=\s*(.*)$", mk, flags=re.M).group(1).split())
    users = set()
    for f in os.listdir(os.path.join(PKG, "csrc")):
        if f.endswith(".hip") and re.search(r"\blds_load(16|4)\s*\(", open(os.path.join(PKG, "csrc", f)).read()):
            users.add("csrc/" + f)
    assert users and users <= checked


def test_the_built_assembly_passes():
    mk = open(os.path.join(PKG, "Makefile")).read()
    srcs = re.search(r"^M0_SRCS\s*=\s*(.*)$", mk, flags=re.M).group(1).split()
    paths = [os.path.join(PKG, "_build", os.path.basename(s)[:-4] + ".s") for s in srcs]
    if not all(os.path.exists(p) for p in paths):
        pytest.skip("no build here (the device assembly is written by make)")
    for p in paths:
        bad, nfunc, pairs = check_m0.check(p)
        assert bad == [] and nfunc > 0 and pairs > 0
