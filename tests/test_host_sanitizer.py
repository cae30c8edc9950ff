"""Host-side AddressSanitizer / UndefinedBehaviorSanitizer run of the C ABI (CPU).

Every source under csrc/ is compiled for gfx950 with the sanitizers on the host
pass only (`-Xarch_host -fsanitize=...`), linked into a shared library, and driven by a
program generated from include/fsi.h that calls every exported entry point with
argument sets that must be rejected or accepted on the host before any launch:
all pointers null with sizes 0, then with sizes -1, then with sizes 1.  The
argument checks, size arithmetic and error-string paths run under ASan / UBSan
(any report aborts the driver); nothing reaches a GPU (HIP_VISIBLE_DEVICES is
empty).  Skipped without hipcc.  The driver is linked by ROCm's clang++, whose
sanitizer runtime the library's host code was built against."""
import os
import re
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "foveal-sparse-indexer_amd" / "csrc"
HEADER = ROOT / "include" / "fsi.h"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CLANGXX = "/opt/rocm/llvm/bin/clang++"


def _decls():
    text = HEADER.read_text()
    out = []
    for ret, name, params in re.findall(r"FSI_API\s+([^;]*?)\b(fsi_\w+)\s*\(([^)]*)\)\s*;", text, re.S):
        ps = [" ".join(p.split()) for p in params.split(",") if p.strip() and p.strip() != "void"]
        out.append((" ".join(ret.split()), name, ps))
    return out


def _arg(param: str, v: int) -> str:
    if "*" in param:
        return "nullptr"
    if param.startswith("float"):
        return f"{float(v)}f"
    if param.startswith("size_t"):
        return "(size_t)0" if v < 0 else f"(size_t){v}"
    return f"({param.rsplit(' ', 1)[0]}){v}"


def _driver(decls) -> str:
    lines = ['#include <cstdio>', '#include <cstdint>', '#include <cstddef>', '#include "fsi.h"', "",
             "int main() {", "  long long acc = 0;"]
    for v in (0, -1, 1):
        for ret, name, ps in decls:
            call = f"{name}({', '.join(_arg(p, v) for p in ps)})"
            if ret.endswith("*"):
                lines.append(f"  {{ const char* s = {call}; acc += s ? (long long)s[0] : 0; }}")
            else:
                lines.append(f"  acc += (long long){call};")
    for code in range(-16, 2):
        lines.append(f"  {{ const char* s = fsi_status_string({code}); acc += s ? (long long)s[0] : 0; }}")
    lines += ['  std::printf("driver done %lld\\n", acc);', "  return 0;", "}"]
    return "\n".join(lines) + "\n"


@pytest.mark.skipif(not (Path(HIPCC).exists() and Path(CLANGXX).exists()), reason="hipcc / ROCm clang++ not available")
def test_c_abi_host_paths_under_asan_ubsan(tmp_path):
    decls = _decls()
    assert len(decls) >= 40
    san = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined", "-Xarch_host",
           "-fno-sanitize-recover=all"]
    flags = ["--offload-arch=gfx950", "-O1", "-g", "-fPIC", "-std=c++17", f"-I{ROOT / 'include'}", *san]
    srcs = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))

    def compile_one(src):
        obj = tmp_path / (src.name + ".o")
        cmd = [HIPCC, *flags, "-c", str(src), "-o", str(obj)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, f"{src.name}: {r.stderr[-2000:]}"
        return obj

    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(compile_one, srcs))
    lib = tmp_path / "libfsi_asan.so"
    r = subprocess.run([HIPCC, "-shared", "-fPIC", *san, "-o", str(lib), *map(str, objs)], capture_output=True,
                       text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    drv = tmp_path / "driver.cpp"
    drv.write_text(_driver(decls))
    exe = tmp_path / "driver"
    r = subprocess.run([CLANGXX, "-std=c++17", "-O0", "-g", "-fsanitize=address,undefined",
                        "-fno-sanitize-recover=all", f"-I{ROOT / 'include'}", str(drv), "-o", str(exe),
                        f"-L{tmp_path}", "-lfsi_asan", f"-Wl,-rpath,{tmp_path}"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1",
               HIP_VISIBLE_DEVICES="")
    r = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    report = r.stdout[-3000:] + r.stderr[-3000:]
    assert r.returncode == 0, report
    assert "driver done" in r.stdout
    assert "AddressSanitizer" not in report and "runtime error" not in report, report
