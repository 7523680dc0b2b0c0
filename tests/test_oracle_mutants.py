"""The oracle's pins are strong enough to catch plausible mistakes.

Each mutant is oracle/mdq_oracle.c with one planted mistake of the kind a restatement of
the reference step could make (a dropped term, a wrong constant, an off-by-one, a transposed
operand, a different rounding or clamp), built into a temporary library.  The oracle's own
pinning tests (closed forms, textbook AdamW, code extremes and ties, tail lanes, the nibble
layout, non-finite rules, Philox known-answer vectors; not the golden fixtures, which the
oracle itself wrote) run against that library in a subprocess and must fail for every mutant,
while the unmodified source passes them.  Only the oracle is mutated, on the CPU."""
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "oracle", "mdq_oracle.c")
PINS = ["tests/test_oracle_step.py", "tests/test_oracle_rounding.py", "tests/test_oracle_nonfinite.py",
        "tests/test_oracle_philox.py::test_philox_kat"]
CFLAGS = ["-O2", "-std=c11", "-fPIC", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", "-march=x86-64-v3"]

# (name, text in mdq_oracle.c, replacement): each text occurs in the source
MUTANTS = [
    ("m moment without (1 - beta1)", "m = fmaf(b1, m, omb1 * g);", "m = fmaf(b1, m, g);"),
    ("v moment with beta1", "v = fmaf(b2, v, (omb2 * g) * g);", "v = fmaf(b1, v, (omb2 * g) * g);"),
    ("v moment without the second g", "v = fmaf(b2, v, (omb2 * g) * g);", "v = fmaf(b2, v, omb2 * fabsf(g));"),
    ("m scale divides by 2^(bits-1) - 1", "(max_m + 1e-12f) / (float)qlm;", "(max_m + 1e-12f) / (float)(qlm - 1.0);"),
    ("v scale divides by 2^bits", "+ 1e-12f) / (float)qlv;", "+ 1e-12f) / (float)(qlv + 1.0);"),
    ("m codes round half to even", "qm = round((double)m / (double)dm);", "qm = nearbyint((double)m / (double)dm);"),
    ("symmetric m clamp", "if (qm < -qlm) qm = -qlm;", "if (qm < 1.0 - qlm) qm = 1.0 - qlm;"),
    ("nibbles transposed", "(uint8_t)((vi << 4) | (mu & 0x0f))", "(uint8_t)((mu << 4) | (vi & 0x0f))"),
    ("m nibble offset 7", "m = ((float)mu - 8.0f) * sm;", "m = ((float)mu - 7.0f) * sm;"),
    ("v dequant without v_min", "v = mdq_oracle_expf(fmaf((float)vq, sv, vmin));",
     "v = mdq_oracle_expf((float)vq * sv);"),
    ("tail lanes left out of the reductions", "float a = 0.0f, l = 0.0f;               /* invalid lanes: :92-93 */",
     "if (idx >= n) continue;\n                float a = 0.0f, l = 0.0f;"),
    ("requant divisor without the 1e-12", "const float dm = s_sm + 1e-12f, dv = s_sv + 1e-12f;",
     "const float dm = s_sm, dv = s_sv;"),
    ("bias correction bc2 not square-rooted", "const float sqrt_bc2 = sqrtf(bc2);", "const float sqrt_bc2 = bc2;"),
    ("weight decay with the wrong sign", "const float decay = 1.0f - lr * wd;", "const float decay = 1.0f + lr * wd;"),
    ("eps left out of the update", "const float denom = sqrtf(v) / sqrt_bc2 + eps;",
     "const float denom = sqrtf(v) / sqrt_bc2;"),
    ("v code from log v without v_min", "qv = round((double)(l - s_vmin) / (double)dv);",
     "qv = round((double)l / (double)dv);"),
    ("Philox multipliers swapped", "(uint64_t)0xD2511F53u * c0;", "(uint64_t)0xCD9E8D57u * c0;"),
    ("stochastic m uniform over [0, 2)", "*um = ((float)(w & 0xffffu) + 0.5f) * (1.0f / 65536.0f);",
     "*um = ((float)(w & 0xffffu) + 0.5f) * (1.0f / 32768.0f);"),
    ("stochastic rounding to nearest of q + u", "qm = (double)floorf(fmaf(m, inv_dm, um));",
     "qm = (double)rintf(fmaf(m, inv_dm, um));"),
    ("stochastic counter without the element offset", "sr_uniforms((uint64_t)(idx + t->elem_offset),",
     "sr_uniforms((uint64_t)idx,"),
    ("stochastic counter without the step", "tensor_id, (uint32_t)step};", "tensor_id, 0u};"),
    ("stochastic counter without the tensor id", "(uint32_t)(idx >> 34), tensor_id,", "(uint32_t)(idx >> 34), 0u,"),
]


def _build(tmp, name, src_text):
    d = os.path.join(tmp, name)
    os.makedirs(d, exist_ok=True)
    c = os.path.join(d, "mdq_oracle.c")
    with open(c, "w") as f:
        f.write(src_text)
    shutil.copy(os.path.join(ROOT, "oracle", "mdq_oracle.h"), d)
    lib = os.path.join(d, "libmdq_oracle.so")
    r = subprocess.run(["gcc", *CFLAGS, "-shared", "-o", lib, c, "-lm"], capture_output=True, text=True)
    assert r.returncode == 0, f"{name}: mutant does not compile:\n{r.stderr[-2000:]}"
    return lib


def _pins_pass(lib):
    env = dict(os.environ, MDQ_ORACLE_LIB=lib, OMP_NUM_THREADS="2")
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider", *PINS],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    return r.returncode == 0, r.stdout[-1500:]


@pytest.mark.slow
def test_every_planted_mistake_fails_the_pinning_tests(tmp_path):
    with open(SRC) as f:
        src = f.read()
    jobs = {}
    for name, old, new in MUTANTS:
        assert src.count(old) >= 1, f"{name}: {old!r} not in mdq_oracle.c"
        jobs[name] = src.replace(old, new, 1)
    jobs["unmodified"] = src
    tmp = str(tmp_path)
    libs = {k: _build(tmp, f"m{i}", v) for i, (k, v) in enumerate(jobs.items())}
    with cf.ThreadPoolExecutor(max_workers=4) as ex:
        res = dict(zip(libs, ex.map(_pins_pass, libs.values())))
    ok, out = res.pop("unmodified")
    assert ok, f"the unmodified oracle fails its pinning tests:\n{out}"
    survivors = [k for k, (passed, _o) in res.items() if passed]
    print(f"{len(res) - len(survivors)} of {len(res)} planted mistakes caught", flush=True)
    assert not survivors, f"mistakes the pinning tests do not catch: {survivors}"
