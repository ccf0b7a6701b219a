"""The public headers as a C caller sees them: every include/*.h compiles as
strict C99 and as C++17 on its own, and a C program links against the built
library and calls into it (no GPU is needed: the device count is 0 here, and
calls without a context fail with ROCKNPU_STATUS_INVALID_ARGUMENT). This is
what a cgo, JNI or other FFI binding of the reference's C ABI compiles
against."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))
LIB = ROOT / "rocknpu_amd" / "librocknpu_capi.so"

pytestmark = pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not installed")


@pytest.mark.parametrize("header", HEADERS, ids=lambda h: h.name)
@pytest.mark.parametrize("lang", [("gcc", "c", "-std=c99"), ("g++", "c++", "-std=c++17")], ids=["c99", "c++17"])
def test_header_compiles_alone(header, lang, tmp_path):
    cc, x, std = lang
    src = tmp_path / "t.src"
    src.write_text(f'#include "{header.name}"\nint rocknpu_header_probe(void) {{ return 0; }}\n')
    r = subprocess.run([cc, "-x", x, std, "-Wall", "-Wextra", "-Werror", "-pedantic", "-fsyntax-only",
                        f"-I{ROOT / 'include'}", str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


C_PROGRAM = r"""
#include <stdio.h>
#include "rocknpu.h"
#include "rocknpu_ggml.h"
#include "rocknpu_route.h"
#include "rocknpu_sidecar.h"
#include "rocknpu_hip.h"

int main(void) {
    float out[4] = {0};
    const float act[4] = {0};
    const uint8_t w[144] = {0};
    int bm = 0, bn = 0, st = 0;
    size_t count = rocknpu_device_count();
    /* a NULL context is an invalid argument, as in the reference */
    int s1 = rocknpu_matmul_q4_k_f32_f32(NULL, w, sizeof w, act, out, 1, 256, 1);
    /* host-only helpers answer without a GPU */
    int s2 = rocknpu_hip_gemm_route(4096, 14336, 4096, 256, &bm, &bn, &st);
    printf("%zu %d %d %d %d %d\n", count, s1, s2, bm, bn, st);
    return 0;
}
"""


@pytest.mark.skipif(not LIB.exists(), reason="library not built")
def test_c_program_links_and_calls(tmp_path):
    src = tmp_path / "caller.c"
    src.write_text(C_PROGRAM)
    exe = tmp_path / "caller"
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", f"-I{ROOT / 'include'}", str(src), "-o", str(exe),
                        f"-L{LIB.parent}", "-lrocknpu_capi", f"-Wl,-rpath,{LIB.parent}",
                        "-Wl,-rpath-link,/opt/rocm/lib", "-Wl,-rpath,/opt/rocm/lib"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    count, s1, s2, bm, bn, st = (int(v) for v in r.stdout.split())
    assert s1 == -1  # ROCKNPU_STATUS_INVALID_ARGUMENT
    assert (s2, bm, bn, st) == (0, 256, 256, 2)
    assert count >= 0


def test_route_stats_layout_matches_the_python_mirror(tmp_path):
    """rocknpu_route_stats as C lays it out equals route.RouteStats (ctypes):
    size and every field's offset."""
    from rocknpu_amd import route
    fields = [name for name, _ in route.RouteStats._fields_]
    src = tmp_path / "layout.c"
    body = "".join(f'    printf("%zu\\n", offsetof(rocknpu_route_stats, {f}));\n' for f in fields)
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "rocknpu_route.h"\nint main(void) {\n'
                   '    printf("%zu\\n", sizeof(rocknpu_route_stats));\n' + body + "    return 0;\n}\n")
    exe = tmp_path / "layout"
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    import ctypes
    want = [ctypes.sizeof(route.RouteStats)] + [getattr(route.RouteStats, f).offset for f in fields]
    assert got == want
