#!/bin/sh
# Builds the CPU oracle (test infrastructure): oracle/_build/librg_cpu.so.
# gcc, no fast math and no floating-point contraction, so every float operation rounds as the
# reference's Rust code does; OpenMP where the reference uses rayon (results do not depend on
# the thread count: task boundaries are fixed, as in src/plan.rs:6-10 and 1396-1399).
set -e
cd "$(dirname "$0")"
mkdir -p _build
g++ -O3 -march=x86-64-v3 -ffp-contract=off -fno-fast-math -fopenmp -std=c++17 -shared -fPIC \
    -Wall -Wno-sign-compare cpu_exec.cpp -o _build/librg_cpu.so
