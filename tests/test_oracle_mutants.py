"""Mutation tests of the CPU oracle: each plausible mistake is planted in the
text of oracle/oracle.c, the mutant is compiled with the oracle's own flags
into a temporary directory, and the pinning checks of test_oracle.py,
test_oracle_decode.py and test_oracle_kquant.py are run against it.  Every
mutant must fail at least one check, and the unmutated source, built the same
way, must pass them all (so the harness itself does not fail everything).
CPU only; needs gcc."""
import inspect
import itertools
import shutil
import subprocess
from pathlib import Path

import pytest

from tests import test_oracle, test_oracle_decode, test_oracle_kquant
from tests._oracle import ORACLE_DIR, Oracle

# (name, text in oracle.c, replacement, occurrence to replace: 1-based, 0 = all)
MUTANTS = [
    ("q4_0 nibble halves swapped in dequantization",
     "int x0 = (int)(qs[j] & 0x0F) - 8;\n      int x1 = (int)(qs[j] >> 4) - 8;\n      out[j] = (float)x0 * d;",
     "int x0 = (int)(qs[j] >> 4) - 8;\n      int x1 = (int)(qs[j] & 0x0F) - 8;\n      out[j] = (float)x0 * d;", 1),
    ("q4_0 -8 offset dropped",
     "int x0 = (int)(qs[j] & 0x0F) - 8;", "int x0 = (int)(qs[j] & 0x0F);", 0),
    ("q4_1 minimum not added", "out[j] = p0 + m;", "out[j] = p0;", 1),
    ("q8_0 quants read unsigned",
     "const int8_t* qs = (const int8_t*)(b + 2);", "const uint8_t* qs = (const uint8_t*)(b + 2);", 1),
    ("f16 exponent bias off by one", "bits = sign | ((exp + 112u) << 23) | (man << 13);",
     "bits = sign | ((exp + 111u) << 23) | (man << 13);", 1),
    ("f16 subnormals mis-normalised", "((uint32_t)(112 - e) << 23)", "((uint32_t)(113 - e) << 23)", 1),
    ("q4_0 scalar GEMV accumulates the high half first",
     "float p0 = w0 * in[j];\n          sum = sum + p0;\n          float p1 = w1 * in[j + 16];\n          sum = sum + p1;",
     "float p1 = w1 * in[j + 16];\n          sum = sum + p1;\n          float p0 = w0 * in[j];\n          sum = sum + p0;", 1),
    ("GEMM reads b transposed", "float p = a[i * k + l] * b[l * n + j];", "float p = a[i * k + l] * b[j * k + l];", 1),
    ("RMSNorm epsilon dropped (f64)", "double rms = sqrt(ss / (double)hidden + eps);",
     "double rms = sqrt(ss / (double)hidden);", 1),
    ("RMSNorm epsilon dropped (f32)", "float rms = sqrtf(mean + eps);", "float rms = sqrtf(mean);", 1),
    ("SiLU with exp(+g)", "float e = expf(-g);", "float e = expf(g);", 1),
    ("RoPE rotation sign", "out[i + h] = x1 * s + x2 * c;", "out[i + h] = x2 * c - x1 * s;", 1),
    ("RoPE frequencies 1/base^(i/d)", "float e = (2.0f * (float)i) / (float)head_dim;",
     "float e = ((float)i) / (float)head_dim;", 1),
    ("q4_k odd scales without their high bits",
     "else scales[i] = (uint8_t)(((b[src] >> 6) | ((b[src + 1] & 15) << 2)) & 63);",
     "else scales[i] = (uint8_t)((b[src] >> 6) & 63);", 1),
    ("q6_k bias -31", "float u = t * (float)((int)(int8_t)q - 32);", "float u = t * (float)((int)(int8_t)q - 31);", 1),
    ("q5 high half takes bit j + 12", "uint32_t xh_1 = (qh >> (j + 12)) & 0x10;",
     "uint32_t xh_1 = ((qh >> (j + 12)) << 4) & 0x10;", 1),
    ("q5 qh read big-endian",
     "uint32_t qh = (uint32_t)qhp[0] | ((uint32_t)qhp[1] << 8) | ((uint32_t)qhp[2] << 16) | ((uint32_t)qhp[3] << 24);",
     "uint32_t qh = (uint32_t)qhp[3] | ((uint32_t)qhp[2] << 8) | ((uint32_t)qhp[1] << 16) | ((uint32_t)qhp[0] << 24);", 1),
    ("q5_0 -16 offset dropped", "out[j] = (float)((int32_t)x0 - 16) * d;", "out[j] = (float)((int32_t)x0) * d;", 1),
    ("q5_1 minimum not added", "out[j + 16] = p1 + m;\n      } else {", "out[j + 16] = p1;\n      } else {", 1),
]

MODULES = (test_oracle, test_oracle_decode, test_oracle_kquant)


def checks():
    """Every oracle check (a test function taking `orc`), with its
    parametrizations expanded: a list of (name, zero-argument callable taking orc)."""
    out = []
    for mod in MODULES:
        for name, fn in sorted(vars(mod).items()):
            if not name.startswith("test_") or not callable(fn):
                continue
            params = list(inspect.signature(fn).parameters)
            if not params or params[0] != "orc":
                continue
            grids = [m for m in getattr(fn, "pytestmark", []) if m.name == "parametrize"]
            axes = []
            for m in grids:
                names = [a.strip() for a in m.args[0].split(",")] if isinstance(m.args[0], str) else list(m.args[0])
                vals = [v if len(names) > 1 else (v,) for v in m.args[1]]
                axes.append([dict(zip(names, v)) for v in vals])
            for combo in itertools.product(*axes) if axes else [()]:
                kw = {}
                for part in combo:
                    kw.update(part)
                if set(kw) | {"orc"} != set(params):
                    continue
                out.append((f"{mod.__name__}.{name}{kw or ''}", lambda orc, fn=fn, kw=kw: fn(orc, **kw)))
    return out


def build(tmp: Path, source: str) -> Path:
    """Compiles oracle.c text `source` (with the unchanged oracle_simd.c and
    oracle.h) into tmp/liboracle.so with the flags of oracle/Makefile."""
    tmp.mkdir(parents=True, exist_ok=True)
    (tmp / "oracle.c").write_text(source)
    for f in ("oracle.h", "oracle_simd.c"):
        shutil.copy(ORACLE_DIR / f, tmp / f)
    cc = ["gcc", "-O2", "-fPIC", "-ffp-contract=off", "-fno-fast-math", "-std=c11", "-w"]
    subprocess.run(cc + ["-c", "-o", str(tmp / "oracle.o"), str(tmp / "oracle.c")], check=True)
    subprocess.run(["gcc", "-O3", "-mavx2", "-mfma", "-fPIC", "-std=c11", "-w", "-pthread", "-c", "-o",
                    str(tmp / "oracle_simd.o"), str(tmp / "oracle_simd.c")], check=True)
    lib = tmp / "liboracle.so"
    subprocess.run(["gcc", "-shared", "-pthread", "-o", str(lib), str(tmp / "oracle.o"), str(tmp / "oracle_simd.o"),
                    "-lm"], check=True)
    return lib


def failing_checks(orc) -> list[str]:
    failed = []
    for name, run in checks():
        try:
            run(orc)
        except Exception:  # an assertion or any error the mistake causes
            failed.append(name)
    return failed


def apply(source: str, old: str, new: str, occurrence: int) -> str:
    n = source.count(old)
    assert n >= max(occurrence, 1), f"mutation site not found ({n} occurrences): {old!r}"
    if occurrence == 0:
        return source.replace(old, new)
    at = -1
    for _ in range(occurrence):
        at = source.index(old, at + 1)
    return source[:at] + new + source[at + len(old):]


def test_unmutated_oracle_passes_every_check(tmp_path):
    orc = Oracle(build(tmp_path / "base", (ORACLE_DIR / "oracle.c").read_text()))
    assert len(checks()) >= 40
    assert failing_checks(orc) == []


@pytest.mark.parametrize("name,old,new,occurrence", MUTANTS, ids=[m[0] for m in MUTANTS])
def test_planted_mistake_fails_a_check(tmp_path, name, old, new, occurrence):
    src = apply((ORACLE_DIR / "oracle.c").read_text(), old, new, occurrence)
    orc = Oracle(build(tmp_path / "mutant", src))
    failed = failing_checks(orc)
    print(f"[mutant] {name}: caught by {len(failed)} checks, e.g. {failed[:3]}")
    assert failed, f"planted mistake '{name}' passes every oracle check"
