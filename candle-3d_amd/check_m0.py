"""Build check for the inline-assembly direct global -> LDS loads
(lds_load16 / lds_load4 in csrc/common.hpp).

Each of those loads is one asm statement holding the pair

    s_mov_b32 m0, <sgpr>
    buffer_load_dword[x4] <vgpr>, <rsrc>, <soffset> offen lds

which overwrites m0 (the LDS destination address) behind the compiler's
back. That is safe only while the compiler keeps nothing of its own in m0
in the same kernel. This script reads the device assembly of a translation
unit (hipcc --cuda-device-only -S) and fails the build when any function in
it breaks that:

  - an instruction outside an inline-asm block names m0 (the compiler set or
    read it for its own use);
  - an inline-asm block that names m0 is anything but exactly that pair;
  - an instruction that uses m0 implicitly appears outside the asm blocks
    (s_sendmsg*, s_ttracedata, s_movrel* / v_movrel*, v_interp*, ds_gws*,
    ds_append / ds_consume / ds_ordered_count, the *_addtid LDS forms, and
    buffer / global loads to LDS).

Usage: python3 check_m0.py FILE.s [FILE.s ...]; exit status 1 with a report
on the first violations, 0 (and one summary line) otherwise.
"""
from __future__ import annotations

import re
import sys

M0 = re.compile(r"\bm0\b")
PAIR_MOV = re.compile(r"^s_mov_b32\s+m0,\s*s\d+$")
PAIR_LOAD = re.compile(r"^buffer_load_dword(x4)?\s+v\d+,\s*s\[\d+:\d+\],\s*(s\d+|\d+)\s+offen\s+lds$")
IMPLICIT = re.compile(r"^(s_sendmsg|s_ttracedata|s_movrel|v_movrel|v_interp|ds_gws|ds_append|ds_consume|"
                      r"ds_ordered_count|ds_read_addtid|ds_write_addtid|ds_load_addtid|ds_store_addtid)"
                      r"|^(buffer|global)_load\S*\s.*\blds\b")
FUNC = re.compile(r"^([A-Za-z_.$][\w.$]*):")


def _instr(line: str) -> str:
    """The instruction text of an assembly line ('' for labels, directives,
    comments and blank lines)."""
    s = line.split(";", 1)[0].strip()
    if not s or s.startswith(".") or s.endswith(":"):
        return ""
    return s


def check(path: str) -> tuple[list[str], int, int]:
    """(violations, functions seen, m0 pairs seen) for one assembly file."""
    bad: list[str] = []
    func = "?"
    nfunc = pairs = 0
    in_asm = False
    block: list[tuple[int, str]] = []
    with open(path) as f:
        for no, raw in enumerate(f, 1):
            line = raw.rstrip("\n")
            m = FUNC.match(line)
            if m and not line.startswith(("\t", " ")) and not m.group(1).startswith(".L"):
                func = m.group(1)
                nfunc += 1
            if ";;#ASMSTART" in line:
                in_asm, block = True, []
                continue
            if ";;#ASMEND" in line:
                in_asm = False
                ins = [(n, s) for n, s in block if s]
                if any(M0.search(s) for _, s in ins):
                    ok = len(ins) == 2 and PAIR_MOV.match(ins[0][1]) and PAIR_LOAD.match(ins[1][1])
                    if ok:
                        pairs += 1
                    else:
                        bad.append(f"{path}:{block[0][0] if block else no}: {func}: inline asm naming m0 is not "
                                   f"the s_mov_b32 m0 + buffer_load ... lds pair: {[s for _, s in ins]}")
                continue
            s = _instr(line)
            if in_asm:
                block.append((no, s))
                continue
            if not s:
                continue
            if M0.search(s):
                bad.append(f"{path}:{no}: {func}: compiler-generated use of m0: {s}")
            elif IMPLICIT.search(s):
                bad.append(f"{path}:{no}: {func}: instruction that uses m0 implicitly: {s}")
    return bad, nfunc, pairs


def main(argv: list[str]) -> int:
    if len(argv) < 2:
        print(__doc__.strip().splitlines()[-2], file=sys.stderr)
        return 2
    failed = False
    for path in argv[1:]:
        bad, nfunc, pairs = check(path)
        if bad:
            failed = True
            print(f"check_m0: {path}: {len(bad)} violation(s)", file=sys.stderr)
            for b in bad[:20]:
                print("  " + b, file=sys.stderr)
        else:
            print(f"check_m0: {path}: ok ({nfunc} functions, {pairs} m0 + LDS-load pairs, no other m0 use)")
    return 1 if failed else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
