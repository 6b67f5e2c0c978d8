"""Mutation check of the oracle's pins -- CPU only.

Builds altered copies of oracle/camelid_oracle.cpp, each with one plausible rewrite of a cited
reference expression (a different association, a division for a reciprocal product, a
contracted multiply-add), and runs the oracle's pin files against each build
(CAMELID_ORACLE_LIB).  Every altered build must fail at least one pin, and the unaltered
source, built the same way, must pass them all.  This is what makes the oracle's arithmetic
"pinned": a slip of any of these kinds in the oracle would not go unnoticed, even though the
GPU kernels are compared against the oracle rather than against the reference itself.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
SRC = ROOT / "oracle" / "camelid_oracle.cpp"
PIN_FILES = ["tests/test_oracle_pins.py", "tests/test_oracle_order_pins.py",
             "tests/test_oracle_elementwise_pins.py"]

# name -> (source text, its rewrite); each source text occurs exactly once in the oracle
MUTANTS = {
    # elementwise expressions (tensor/mod.rs, inference.rs, rope.rs citations in the oracle)
    "swiglu: g * (u / (1 + exp(-g)))":
        ("return (g / (1.0f + std::exp(-g))) * u;", "return g * (u / (1.0f + std::exp(-g)));"),
    "rmsnorm out: x * (scale * w)":
        ("out[i] = (x[i] * scale) * w[i];", "out[i] = x[i] * (scale * w[i]);"),
    "rmsnorm scale: sqrt(1 / (ms + eps))":
        ("float scale = 1.0f / std::sqrt(ms + eps);", "float scale = std::sqrt(1.0f / (ms + eps));"),
    "rmsnorm mean: ss * (1 / n)":
        ("float ms = ss / (float)n;", "float ms = ss * (1.0f / (float)n);"),
    "softmax: e / sum":
        ("float prob = sc[p] * inv;", "float prob = sc[p] / sum;"),
    "score: dot / sqrt(hd)":
        ("sc[p] = dot_product(qh, &m.kc[base + (size_t)p * m.hd], m.hd) * scale;",
         "sc[p] = dot_product(qh, &m.kc[base + (size_t)p * m.hd], m.hd) / std::sqrt((float)m.hd);"),
    "rope rotation: fma(x0, c, -(x1 s))":
        ("data[d0] = (x0 * c) - (x1 * s);", "data[d0] = std::fma(x0, c, -(x1 * s));"),
    "rope rotation: fma(-x1, s, x0 c)":
        ("data[d0] = (x0 * c) - (x1 * s);", "data[d0] = std::fma(-x1, s, x0 * c);"),
    "rope frequency: 1 / powf(base, 2i/d)":
        ("float base = std::pow(c.freq_base, -((float)pair * 2.0f) / (float)c.rope_dim);",
         "float base = 1.0f / std::pow(c.freq_base, ((float)pair * 2.0f) / (float)c.rope_dim);"),
    "llama3: (1 - smooth) * (f / factor)":
        ("return ((1.0f - smooth) * frequency / c.factor) + (smooth * frequency);",
         "return ((1.0f - smooth) * (frequency / c.factor)) + (smooth * frequency);"),
    "q8_0 quantize: x / unrounded":
        ("float r = std::round(block[i] * inv);",
         "float r = std::round(unrounded == 0.0f ? 0.0f : block[i] / unrounded);"),
    "q8_0 scale: amax * (1 / 127)":
        ("float unrounded = max_abs / 127.0f;", "float unrounded = max_abs * (1.0f / 127.0f);"),
    "q8_0 quantize: inverse of the f16-rounded scale":
        ("float inv = (unrounded == 0.0f) ? 0.0f : 1.0f / unrounded;",
         "float inv = (unrounded == 0.0f) ? 0.0f : 1.0f / *scale_out;"),
    "q8_k scale: max / -127":
        ("*d = 1.0f / iscale;", "*d = mx / -127.0f;"),
    "q8_k quants: (-127 x) / max":
        ("qs[i] = (int8_t)std::min(nearest_int(iscale * x[i]), 127);",
         "qs[i] = (int8_t)std::min(nearest_int((-127.0f * x[i]) / mx), 127);"),
    # reductions (order pins)
    "q8_0 row fold: fused multiply-add":
        ("sum += ((float)d * ws) * xs[b];", "sum = std::fma((float)d * ws, xs[b], sum);"),
    "q8_0 row fold: w_d * x_d first":
        ("sum += ((float)d * ws) * xs[b];", "sum += (float)d * (ws * xs[b]);"),
    "rmsnorm sum: fused multiply-add":
        ("for (size_t i = 0; i < n; ++i) ss += x[i] * x[i];",
         "for (size_t i = 0; i < n; ++i) ss = std::fma(x[i], x[i], ss);"),
    "rmsnorm sum: reversed":
        ("for (size_t i = 0; i < n; ++i) ss += x[i] * x[i];",
         "for (size_t i = n; i-- > 0;) ss += x[i] * x[i];"),
    "score dot: fused multiply-add":
        ("for (size_t i = 0; i < n; ++i) sum += a[i] * b[i];",
         "for (size_t i = 0; i < n; ++i) sum = std::fma(a[i], b[i], sum);"),
    "attention AV: fused multiply-add":
        ("for (uint32_t d = 0; d < m.hd; ++d) out[d] += prob * vr[d];",
         "for (uint32_t d = 0; d < m.hd; ++d) out[d] = std::fma(prob, vr[d], out[d]);"),
}


def _build(src_text: str, out: Path) -> None:
    cpp = out.with_suffix(".cpp")
    cpp.write_text(src_text)
    subprocess.run(["g++", "-O3", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-fPIC", "-shared",
                    "-o", str(out), str(cpp), "-lm"], check=True)


def _run_pins(lib: Path) -> int:
    env = dict(os.environ, CAMELID_ORACLE_LIB=str(lib), OMP_NUM_THREADS="1")
    proc = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-m", "not gpu", *PIN_FILES],
                          cwd=ROOT, env=env, capture_output=True, text=True)
    return proc.returncode


def test_every_mutant_fails_a_pin_and_the_source_passes(tmp_path):
    orig = SRC.read_text()
    jobs = {"(unaltered)": orig}
    for i, (name, (a, b)) in enumerate(MUTANTS.items()):
        assert orig.count(a) == 1, f"mutation site not unique or missing: {name}"
        jobs[name] = orig.replace(a, b)

    def one(item):
        k, (name, text) = item
        lib = tmp_path / f"m{k}.so"
        _build(text, lib)
        return name, _run_pins(lib)

    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as pool:
        rcs = dict(pool.map(one, enumerate(jobs.items())))
    assert rcs.pop("(unaltered)") == 0
    # pytest exit code 1 = tests ran and some failed (2+ would be an error, not a caught mutant)
    survivors = {n: rc for n, rc in rcs.items() if rc != 1}
    assert not survivors, f"mutants not caught by any pin: {survivors}"
