"""The oracle's pins catch plausible mistakes.

Each case plants one mistake in a scratch copy of oracle/mimref.c (a dropped
term, a swapped nibble order, a wrong scale index, an f32 quotient in place of
the f64 one, ...), builds it, and runs the oracle tests against it through
MIMREF_LIB in a subprocess. The tests must fail. CPU only; the product is
never touched.
"""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "oracle", "mimref.c")

# (name, original text, planted text, tests expected to catch it)
MUTATIONS = [
    ("q4k_nibble_swap",
     "y[64 * c + l] = d1 * (float)(q[32 * c + l] & 0xF) - m1;",
     "y[64 * c + l] = d1 * (float)(q[32 * c + l] >> 4) - m1;",
     "test_dequantize_golden"),
    ("q4k_min_high_bits",
     "*m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));",
     "*m = (uint8_t)((q[j + 4] >> 4) | ((q[j - 4] >> 6) << 4));",
     "test_dequantize_golden"),
    ("q6k_decode_scale_index",
     "float s = d * (float)sc[8 * h + is + 2 * p];",
     "float s = d * (float)sc[8 * h + is + p];",
     "test_dequantize_golden"),
    ("q6k_offset",
     "return v - 32;",
     "return v - 31;",
     "test_dequantize_golden"),
    ("q4k_dot_drops_min_term",
     "*out = tot - off;",
     "*out = tot;",
     "test_dot_a8k_closed_form"),
    ("q6k_dot_scale_index",
     "S += (int32_t)sc[8 * h + is + 2 * p] * q6_quant(blk, h, p, l) * y[128 * h + 32 * p + l];",
     "S += (int32_t)sc[8 * h + is + p] * q6_quant(blk, h, p, l) * y[128 * h + 32 * p + l];",
     "test_dot_a8k_closed_form"),
    ("act_quant_f32_quotient",
     "nearbyint(127.0 * (double)xb[i] / (double)amax)",
     "nearbyint((double)(127.0f * xb[i] / amax))",
     "test_quantize_act_exact_rounding or test_quantize_act_known_answers"),
    ("f16_subnormal_shift",
     "return bits_f32(sign | e << 23 | (mant & 0x3FFu) << 13);",
     "return bits_f32(sign | e << 23 | (mant & 0x3FFu) << 12);",
     "test_f16_to_f32_exhaustive"),
]


@pytest.mark.parametrize("name,orig,planted,tests", MUTATIONS, ids=[m[0] for m in MUTATIONS])
def test_mutation_is_caught(tmp_path, name, orig, planted, tests):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    src = open(SRC).read()
    assert src.count(orig) == 1, f"mutation site of {name} not found once in mimref.c"
    d = tmp_path / name
    d.mkdir()
    (d / "mimref.c").write_text(src.replace(orig, planted))
    shutil.copy(os.path.join(ROOT, "oracle", "mimref.h"), d / "mimref.h")
    lib = d / "libmimref.so"
    subprocess.run(["gcc", "-O2", "-mavx2", "-mfma", "-ffp-contract=off", "-fno-fast-math", "-fPIC",
                    "-fopenmp", "-shared", "-o", str(lib), str(d / "mimref.c"), "-lm"], check=True)
    env = dict(os.environ, MIMREF_LIB=str(lib))
    r = subprocess.run([sys.executable, "-m", "pytest", os.path.join(ROOT, "tests", "test_oracle.py"),
                        "-x", "-q", "-p", "no:cacheprovider", "-k", tests],
                       env=env, cwd=ROOT, capture_output=True, text=True, timeout=600)
    assert r.returncode == 1, f"{name} not caught by {tests}:\n{r.stdout[-2000:]}"
