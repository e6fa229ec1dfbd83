"""Compile the HIP smoke programs (tests/smoke/*.cpp) into tests/smoke/bin/.

They link liboperatorlib.so (the product, through its C++ API) and
oracle/liboracle.so (the checker). Both must be built first; the driver's
``__graft_entry__.build()`` does that in order. Run-time library paths are
relative ($ORIGIN), so the binaries work wherever the repository is copied.
"""

from __future__ import annotations

import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
BIN = HERE / "bin"
sys.path.insert(0, str(REPO / "orin-cuda-operator-library_amd"))

from operatorlib import _build  # noqa: E402

ORACLE = REPO / "oracle"


def programs() -> list[Path]:
    return sorted(BIN / src.stem for src in HERE.glob("*.cpp"))


def build(verbose: bool = False) -> list[Path]:
    BIN.mkdir(exist_ok=True)
    lib_rel = "$ORIGIN/../../../orin-cuda-operator-library_amd/operatorlib/lib"
    oracle_rel = "$ORIGIN/../../../oracle"

    def one(src: Path) -> Path:
        exe = BIN / src.stem
        cmd = [_build.HIPCC, *_build.COMMON_FLAGS, "-I", str(ORACLE), str(src),
               f"-L{_build.LIB_DIR}", "-loperatorlib", f"-L{ORACLE}", "-loracle",
               f"-Wl,-rpath,{lib_rel}:{oracle_rel}", "-o", str(exe)]
        if verbose:
            print(" ".join(cmd), flush=True)
        proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"smoke build failed: {src.name}\n{proc.stdout}")
        return exe

    with ThreadPoolExecutor(4) as pool:
        return list(pool.map(one, sorted(HERE.glob("*.cpp"))))


if __name__ == "__main__":
    for exe in build(verbose="-v" in sys.argv):
        print(f"built {exe.relative_to(REPO)}")
