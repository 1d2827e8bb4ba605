"""Pass 1 of the panel SpMV (``panel_products`` in csr_panel.hip) stages its
panel of x with buffer-to-LDS loads issued before the chunk's prefetch
loads, then waits with ``s_waitcnt vmcnt(N)``, N = the prefetch loads
issued after the panel: loads complete in order, so that wait covers the
panel alone.  This holds only if the compiler keeps the panel loads first
and emits exactly N vector loads between them and the wait, so the test
compiles the kernel to gfx950 assembly (no GPU needed) and checks, for each
variant that stages directly (float32, complex64; products and the x-only
gather of the value gradient):

- a buffer-to-LDS load (``buffer_load_dwordx4 ... lds``) comes before the
  first other vector load;
- the vector loads between them and the first barrier number exactly N;
- the last wait before that barrier is ``s_waitcnt vmcnt(N)``.
"""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "mlx-sparse_amd" / "csrc"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

# (value type, x-only) -> prefetch loads after the panel: 8 quads of values
# (one 16-byte load each, two for complex64) and of columns, or columns only
EXPECTED = {("F32", 0): 16, ("F32", 1): 8, ("C64", 0): 24, ("C64", 1): 8}


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    if not Path(HIPCC).exists():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("isa") / "csr_panel.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           f"-I{ROOT / 'include'}", f"-I{CSRC}", "--cuda-device-only", "-S",
           "-o", str(out), str(CSRC / "csr_panel.hip")]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr
    return out.read_text().split("\n")


def _functions(lines):
    """{mangled name: body lines} of every panel_products instantiation."""
    out, cur = {}, None
    for line in lines:
        m = re.match(r"^(_ZN3msx12_GLOBAL__N_114panel_products\S*):", line)
        if m:
            cur = m.group(1)
            out[cur] = []
            continue
        if cur is not None:
            if "s_endpgm" in line:
                cur = None
            else:
                out[cur].append(line)
    return out


@pytest.mark.parametrize("vt,xonly", sorted(EXPECTED))
def test_panel_loads_first_and_wait_counts_prefetch(asm, vt, xonly):
    funcs = _functions(asm)
    tag = f"panel_productsINS_3{vt}ELb{xonly}E"
    names = [n for n in funcs if tag in n]
    assert len(names) == 1, (tag, list(funcs))
    body = funcs[names[0]]
    vload = [i for i, line in enumerate(body)
             if re.search(r"\b(buffer|global)_load_", line)]
    lds = [i for i in vload if "lds" in body[i].split(";")[0]]
    assert lds, "no buffer-to-LDS load"
    first_other = min(i for i in vload if i not in lds)
    assert max(lds) < first_other, "a prefetch load precedes the panel's loads"
    barrier = next(i for i, line in enumerate(body) if "s_barrier" in line)
    between = [i for i in vload if max(lds) < i < barrier]
    n = EXPECTED[(vt, xonly)]
    assert len(between) == n, (len(between), n)
    waits = [body[i].strip() for i in range(max(lds), barrier) if "s_waitcnt" in body[i]]
    assert waits and waits[-1] == f"s_waitcnt vmcnt({n})", waits
