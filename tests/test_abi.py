"""The C ABI without a GPU: the built ``libmi355.so`` loads and exports every entry point ``include/*.h`` declares;
host-only entry points (pack sizes, launch plans, argument validation) behave; the ctypes signature table covers
the header."""

import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", text))
    return names


def test_header_declares_entry_points():
    names = declared()
    assert {"mi_gemv", "mi_dequant", "mi_malloc", "mi_graph_launch"} <= names


def test_library_exports_every_declared_symbol():
    from monolith_mi355.runtime import hip
    lib = hip.load()
    missing = [n for n in sorted(declared()) if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_table_covers_header():
    from monolith_mi355.runtime import hip
    assert declared() == set(hip.SIGNATURES), declared() ^ set(hip.SIGNATURES)


def test_pack_bytes_matches_host_pack():
    from monolith_mi355.formats import pack as P
    from monolith_mi355.runtime import hip
    lib = hip.load()
    for fmt, fid in hip.MI_FMT.items():
        for n, k in ((37, 512), (17408, 5120), (5120, 17408)):
            assert lib.mi_pack_bytes(fid, n, k) == P.pack_bytes(fmt, n, k)
    assert lib.mi_pack_bytes(1, 16, 100) == 0            # K not a multiple of the chunk


def _desc(hip, **kw):
    base = dict(format=1, n=17408, k=5120, m=1, w=256, x=256, ldx=5120, y=256, ldy=17408)
    base.update(kw)
    return hip.MiGemvDesc(**base)


@pytest.mark.parametrize("n,k,m", [(34816, 5120, 1), (5120, 17408, 1), (34816, 5120, 8), (5120, 17408, 8),
                                   (4096, 4096, 1), (1024, 2048, 16), (16, 128, 3), (5120, 17408, 2)])
def test_gemv_plans_fit_the_hardware(n, k, m):
    from monolith_mi355.runtime import hip
    out = (C.c_int32 * 7)()
    hip.call("mi_gemv_plan", C.byref(_desc(hip, n=n, k=k, m=m, ldx=k, ldy=n)), out)
    kernel, waves, kw, tb, ks, lds, wgs = list(out)
    chunks = k // 128
    # gemv_row (VALU) for M <= 2; gemv_rowm (MFMA, 4-chunk K slices) above when its slices fit, else gemv_tk
    assert kernel == (1 if m <= 2 else 3 if chunks % 4 == 0 else 2)
    assert 1 <= waves <= 16 and kw >= 1 and lds <= 160 * 1024 and wgs >= 1 and ks >= 1 and tb >= 1
    if kernel == 1:                                      # K splits of ≤ waves·kw chunks each
        assert kw in (4, 8, 16) and waves * kw * ks >= chunks
    elif kernel == 3:                                    # 4 chunks per wave, ≤ 12 waves per K split
        assert waves * 4 == kw and waves <= 12 and ks * kw >= chunks and (ks - 1) * kw < chunks
        assert tb * wgs >= -(-n // 16) * ks              # tiles per workgroup × workgroups cover every tile
    else:
        assert ks * kw >= chunks and (ks - 1) * kw < chunks
    ws = hip.load().mi_gemv_workspace_bytes(C.byref(_desc(hip, n=n, k=k, m=m, ldx=k, ldy=n)))
    assert (ws > 0) == (ks > 1)


def test_gemv_rejects_bad_descriptors_before_launch():
    from monolith_mi355.runtime import hip
    lib = hip.load()
    bad = [dict(format=9), dict(k=100), dict(m=0), dict(m=17), dict(ldx=64), dict(w=0), dict(x=8),
           dict(epilogue=1, residual=0), dict(epilogue=2, n=40, ldy=20), dict(ldy=16)]
    for kw in bad:
        assert lib.mi_gemv(C.byref(_desc(hip, **kw)), None) == 1, kw      # MI_E_INVALID, nothing enqueued
        assert hip.last_error().startswith("mi_gemv")


def test_ctypes_descriptors_match_the_header_layout(tmp_path):
    """Every ctypes mirror of a header struct has the C layout: each field's offset and the struct's size, from a
    small program compiled against ``include/lithos_mi355.h`` (a descriptor shorter than the C struct would let the
    library read past it)."""
    import shutil
    import subprocess
    from monolith_mi355.runtime import hip
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    classes = [v for k, v in vars(hip).items()
               if isinstance(v, type) and issubclass(v, C.Structure) and k.startswith("Mi")]
    assert len(classes) >= 15

    def c_name(cls):
        return "mi" + re.sub(r"([A-Z])", lambda m: "_" + m.group(1).lower(), cls.__name__[2:])

    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{ROOT / "include" / "lithos_mi355.h"}"',
             "int main(void) {"]
    for cls in classes:
        n = c_name(cls)
        lines.append(f'  printf("{cls.__name__} size %zu\\n", sizeof({n}));')
        for f, _ in cls._fields_:
            lines.append(f'  printf("{cls.__name__} {f} %zu\\n", offsetof({n}, {f}));')
    lines.append("  return 0;\n}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run([cc, "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True, capture_output=True)
    want = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        cls_name, field, value = line.split()
        want[(cls_name, field)] = int(value)
    for cls in classes:
        assert C.sizeof(cls) == want[(cls.__name__, "size")], (cls.__name__, C.sizeof(cls))
        for f, _ in cls._fields_:
            assert getattr(cls, f).offset == want[(cls.__name__, f)], (cls.__name__, f)
