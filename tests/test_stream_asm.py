"""The streamed matrix-core conv (csrc/conv.hip, conv_igemm_stream) issues
its main-loop loads as inline assembly and waits on the vector-memory
counter itself; the compiler does not know those loads are asynchronous.
Its correctness therefore rests on a property of the generated code: no
compiler-placed instruction touches a register an assembly load writes
before the assembly wait that covers it (a copy, spill or reuse of such a
register would read or clobber it before the data lands).  This test
compiles conv.hip for gfx950 and checks that property on every
instantiation of the kernel.  CPU only (needs hipcc)."""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / 'mlx-lattice_amd' / 'csrc'


def _hipcc():
    for cand in ('/opt/rocm/bin/hipcc', shutil.which('hipcc')):
        if cand and Path(cand).exists():
            return cand
    return None


def _regs(text: str) -> set[int]:
    out: set[int] = set()
    for m in re.finditer(r'v\[(\d+):(\d+)\]|v(\d+)\b', text):
        if m.group(3):
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def pending_register_touches(lines: list[str]) -> list[str]:
    """Compiler instructions that read or write a VGPR whose assembly load
    (between ;;#ASMSTART / ;;#ASMEND) has not yet been followed by an
    assembly s_waitcnt vmcnt."""
    pending: set[int] = set()
    in_asm = False
    bad = []
    for line in lines:
        s = line.strip()
        if s.startswith(';;#ASMSTART'):
            in_asm = True
            continue
        if s.startswith(';;#ASMEND'):
            in_asm = False
            continue
        if not s or s.startswith(';') or s.startswith('.'):
            continue
        op = s.split()[0]
        rest = s[len(op):].split(';')[0]
        if in_asm:
            if op.startswith('buffer_load') and ' lds' not in rest:
                pending |= _regs(rest.split(',')[0])
            elif op == 's_waitcnt' and 'vmcnt' in rest:
                pending.clear()
            continue
        if op != 's_waitcnt' and _regs(rest) & pending:
            bad.append(s)
    return bad


def test_pending_register_checker_flags_a_copy():
    lines = [';;#ASMSTART', 'buffer_load_dwordx4 v[8:11], v2, s[4:7], 0 offen', ';;#ASMEND',
             'v_mov_b32_e32 v20, v9',
             ';;#ASMSTART', 's_waitcnt vmcnt(0)', ';;#ASMEND',
             'v_mov_b32_e32 v21, v10']
    assert pending_register_touches(lines) == ['v_mov_b32_e32 v20, v9']


@pytest.mark.skipif(_hipcc() is None, reason='hipcc is not installed')
def test_stream_kernel_never_touches_pending_load_registers(tmp_path):
    out = tmp_path / 'conv.s'
    subprocess.run([_hipcc(), '--offload-arch=gfx950', '-O3', '-std=c++17', '-Xclang', '-target-feature',
                    '-Xclang', '-packed-fp32-ops', f'-I{ROOT / "include"}', f'-I{CSRC}', '--offload-device-only',
                    '-S', str(CSRC / 'conv.hip'), '-o', str(out)], check=True, capture_output=True)
    lines = out.read_text().split('\n')
    starts = [i for i, l in enumerate(lines) if l.startswith('_Z') and 'conv_igemm_stream' in l.split(':')[0]]
    assert len(starts) >= 16, 'every (dtype, shape, chunk count) instantiation is compiled'
    for st in starts:
        en = next(i for i in range(st, len(lines)) if lines[i].startswith('.Lfunc_end'))
        body = lines[st:en]
        assert any('offen lds' in l for l in body), 'the kernel copies A into LDS'
        bad = pending_register_touches(body)
        assert not bad, (lines[st].split(':')[0], bad[:5])
