#!/usr/bin/env bash
# Standalone runner: the modes of the reference's tools/run_final_standalone.sh
# (compile | smoke | benchmark | all), one operatorlib_run invocation per
# operator, key=value output. `smoke` uses the reference's smoke shapes
# (run_final_standalone.sh:46-64), `benchmark` its benchmark shapes (:66-87).
# The reference's Jetson clock check has no MI355X counterpart; the device
# name is printed by every run instead.
set -euo pipefail

PKG=$(cd "$(dirname "${BASH_SOURCE[0]}")/.." && pwd)
REPO=$(cd "$PKG/.." && pwd)
RUN="$PKG/operatorlib/lib/operatorlib_run"
MODE=${1:-smoke}

compile_all() {
    python3 -c "import sys; sys.path.insert(0, '$PKG'); import operatorlib; operatorlib.build()"
}

run_smoke() {
    "$RUN" reduce --n=1000 --warmup=2 --repeat=5
    "$RUN" softmax --rows=17 --cols=1003 --extreme --warmup=2 --repeat=5
    "$RUN" transpose --rows=1000 --cols=1023 --warmup=2 --repeat=5
    "$RUN" rmsnorm --tokens=17 --hidden=1003 --warmup=2 --repeat=5
    "$RUN" gemm_f32 --m=37 --n=65 --k=1003 --warmup=2 --repeat=5
    "$RUN" gemm_f16 --m=37 --n=65 --k=1003 --warmup=2 --repeat=5
    "$RUN" attention_f32 --b=1 --h=2 --s=37 --d=71 --causal=1 --extreme=1 --warmup=2 --repeat=5
    "$RUN" attention_f16 --b=1 --h=2 --s=37 --d=71 --causal=1 --extreme=1 --warmup=2 --repeat=5
}

run_benchmark() {
    printf 'source_commit=%s\n' "$(git -C "$REPO" rev-parse HEAD 2>/dev/null || echo unknown)"
    "$RUN" reduce --n=16777216 --warmup=10 --repeat=30
    "$RUN" softmax --rows=4096 --cols=1024 --warmup=20 --repeat=50
    "$RUN" transpose --rows=4096 --cols=4096 --warmup=10 --repeat=30
    "$RUN" rmsnorm --tokens=2048 --hidden=4096 --warmup=10 --repeat=30
    "$RUN" gemm_f32 --m=4096 --n=4096 --k=4096 --warmup=5 --repeat=15
    "$RUN" gemm_f16 --m=4096 --n=4096 --k=4096 --warmup=5 --repeat=15
    "$RUN" attention_f32 --b=1 --h=12 --s=1024 --d=128 --causal=0 --warmup=5 --repeat=15
    "$RUN" attention_f16 --b=1 --h=12 --s=1024 --d=128 --causal=0 --warmup=5 --repeat=15
}

case "$MODE" in
    compile) compile_all ;;
    smoke) run_smoke ;;
    benchmark) run_benchmark ;;
    all) compile_all; run_smoke; run_benchmark ;;
    *) printf 'Usage: %s [compile|smoke|benchmark|all]\n' "$0" >&2; exit 2 ;;
esac
