"""Host-side AddressSanitizer check of the C-ABI (development container,
CPU only).

``python -m int_crush_converter_amd.asan_check`` builds a variant of
``libicq.so`` whose host code (argument checks, error strings, launch
set-up, the loader's view of the exports) is compiled with AddressSanitizer
and whose device code is built as usual, then runs ``tests/test_abi.py``
against it with the sanitizer runtime preloaded.  The GPU box never builds
or loads this variant.
"""

from __future__ import annotations

import os
import subprocess
import sys

from . import build as B

ASAN_BUILD = os.path.join(B.BUILD, "asan")
ASAN_LIB = os.path.join(ASAN_BUILD, "libicq_asan.so")
# every sanitizer flag is host-only (-Xarch_host applies to the next option)
COMPILE = ("-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer")
LINK = ("-Xarch_host", "-fsanitize=address", "-shared-libasan")


def runtime() -> str:
    r = subprocess.run([B._hipcc(), "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    path = r.stdout.strip()
    if r.returncode != 0 or not os.path.isabs(path) or not os.path.exists(path):
        raise RuntimeError("the compiler's AddressSanitizer runtime was not found")
    return path


def main(verbose: bool = False) -> int:
    lib = B.build(verbose=verbose, build_dir=ASAN_BUILD, lib=ASAN_LIB, extra=COMPILE, link_extra=LINK)
    root = os.path.dirname(B.PKG)
    env = dict(os.environ)
    env["LD_PRELOAD"] = ":".join(p for p in (runtime(), env.get("LD_PRELOAD", "")) if p)
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1"
    env["IC_LIBICQ_PATH"] = lib
    cmd = [sys.executable, "-m", "pytest", os.path.join(root, "tests", "test_abi.py"), "-q", "-m", "not gpu",
           "-p", "no:cacheprovider"]
    print("running", " ".join(cmd), "with", lib, flush=True)
    return subprocess.run(cmd, cwd=root, env=env).returncode


if __name__ == "__main__":
    sys.exit(main(verbose="-v" in sys.argv))
