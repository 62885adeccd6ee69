"""Shows that the oracle's pinning tests have teeth.

Each case plants one plausible mistake in a copy of the oracle's C source (a dropped term, a
wrong rounding mode, a transposed operand, a reordered fold, a wrong tie rule), compiles the
copy into a temporary library, and checks that the named pinning tests of test_oracle.py fail
against it. The planted text must occur exactly once in the source, so that a case cannot
silently stop planting anything. Every planted mistake keeps its memory accesses in bounds.
Everything here runs on the CPU.
"""
import ctypes as C
import functools
import os
import shutil
import subprocess
import sys

import pytest

import test_oracle as T
import test_oracle_attention as TA

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE = os.path.join(os.path.dirname(HERE), "oracle")
sys.path.insert(0, os.path.dirname(HERE))
from oracle import oracle as O  # noqa: E402

# (name, original text, planted text, pinning tests expected to fail)
MUTATIONS = [
    ("f16 rounds half up",
     "if (rem > 0x1000 || (rem == 0x1000 && (r & 1) == 1)) r += 1;",
     "if (rem >= 0x1000) r += 1;",
     [T.test_f32_to_f16_round_to_nearest_even_against_numpy, T.test_f16_reference_known_answers]),
    ("f16 subnormal exponent off by one",
     "bits = sign | ((113 - shift) << 23) | (m << 13);",
     "bits = sign | ((112 - shift) << 23) | (m << 13);",
     [T.test_f16_to_f32_exhaustive_against_numpy]),
    ("Q4 nibble halves swapped",
     "out[b * QK + j] = (float)((int)(q & 15) - 8) * d;\n            out[b * QK + j + 16] = (float)((int)(q >> 4) - 8) * d;",
     "out[b * QK + j] = (float)((int)(q >> 4) - 8) * d;\n            out[b * QK + j + 16] = (float)((int)(q & 15) - 8) * d;",
     [T.test_q4_all_nibbles_block_known_answer]),
    ("Q4 f32 dot drops the high nibbles",
     "s += lo + hi;",
     "s += lo;",
     [T.test_q4_dots_against_f64_brute_force]),
    ("Q8 quantisation rounds half to even",
     "sat_i8(roundf(xs[j] * id))",
     "sat_i8(rintf(xs[j] * id))",
     [T.test_quantize_q8_0_rounds_half_away_from_zero]),
    ("Q8 block maximum without the absolute value",
     "amax = fmaxf(amax, fabsf(xs[j]));",
     "amax = fmaxf(amax, xs[j]);",
     [T.test_quantize_q8_0_invariants]),
    ("Q4xQ8 block sum with a transposed activation operand",
     "sumi += ((int32_t)(b >> 4) - 8) * (int32_t)(int8_t)x[18 + j];",
     "sumi += ((int32_t)(b >> 4) - 8) * (int32_t)(int8_t)x[2 + j];",
     [functools.partial(T.test_q8_dot_matches_exact_integer_reference, k=256)]),
    ("Q8 dot accumulated in f64",
     "    float acc = 0.0f;\n    for (size_t b = 0; b < k / QK; ++b) {\n        const uint8_t *w = row + b * Q4_BLOCK;",
     "    double acc = 0.0;\n    for (size_t b = 0; b < k / QK; ++b) {\n        const uint8_t *w = row + b * Q4_BLOCK;",
     [T.test_q8_dot_scalar_is_the_block_order_fold]),
    ("router GEMV folded in reverse",
     "for (size_t i = 0; i < k; ++i) s += row[i] * x[i];",
     "for (size_t i = k; i-- > 0;) s += row[i] * x[i];",
     [T.test_matvec_is_a_sequential_f32_fold]),
    ("RMS norm without eps",
     "float scale = 1.0f / sqrtf(mean + eps);",
     "float scale = 1.0f / sqrtf(mean);",
     [T.test_rms_norm_known_answers]),
    ("GELU with a flipped tanh sign",
     "return 0.5f * x * (1.0f + tanhf(inner));",
     "return 0.5f * x * (1.0f - tanhf(inner));",
     [T.test_gelu_fixture_and_limits]),
    ("softmax never normalised",
     "for (size_t i = 0; i < n; ++i) x[i] *= inv;",
     "(void)inv;",
     [T.test_softmax_fixture]),
    ("top-k ties go to the higher index",
     "if (best == n || total_key(x[i]) > total_key(x[best])) best = i;",
     "if (best == n || total_key(x[i]) >= total_key(x[best])) best = i;",
     [T.test_top_k_ties_and_total_order]),
    ("total order without the negative flip",
     "i ^= (int32_t)(((uint32_t)(i >> 31)) >> 1);",
     "(void)0;",
     [T.test_top_k_ties_and_total_order]),
    ("routing-weight clamp dropped",
     "sum = fmaxf(sum, ROUTER_SUM_MIN);",
     "(void)ROUTER_SUM_MIN;",
     [T.test_select_experts_known_answers]),
    ("plan fills its groups in reverse pair order (an unstable sort)",
     "for (size_t i = 0; i < pairs; ++i) {\n        uint32_t k = fill[ids[i]]++;",
     "for (size_t i = pairs; i-- > 0;) {\n        uint32_t k = fill[ids[i]]++;",
     [T.test_moe_plan_is_a_stable_sort]),
    ("GeGLU with gate and up exchanged",
     "h[k * ff + j] = orc_gelu(gu[k * gu_rows + j]) * gu[k * gu_rows + ff + j];",
     "h[k * ff + j] = orc_gelu(gu[k * gu_rows + ff + j]) * gu[k * gu_rows + j];",
     [T.test_experts_q8_against_f64_pipeline]),
    ("combine with reassociated scale and weight",
     "for (size_t i = 0; i < d; ++i) o[i] += yy[i] * ds * wt;",
     "for (size_t i = 0; i < d; ++i) o[i] += yy[i] * (ds * wt);",
     [T.test_experts_q8_against_f64_pipeline]),
    ("Q8 f32 dot reads the quants unsigned",
     "s += (float)(int8_t)blk[2 + j] * xs[j];",
     "s += (float)blk[2 + j] * xs[j];",
     [TA.test_q8_dot_exact_cases, TA.test_q8_dot_and_axpy_against_f64]),
    ("Q8 axpy drops the weight",
     "float d = orc_f16_to_f32(le16(blk)) * w;",
     "float d = orc_f16_to_f32(le16(blk));",
     [TA.test_q8_dot_and_axpy_reference_known_answers, TA.test_q8_dot_and_axpy_against_f64]),
    ("attention window one key too wide",
     "(pos + 1 > win ? pos + 1 - win : 0)",
     "(pos + 1 > win ? pos - win : 0)",
     [TA.test_attention_against_exact_f64, TA.test_attention_fixed_cases]),
    ("attention maps query heads to kv heads round-robin",
     "size_t g = h / (nh / nkv);",
     "size_t g = h % nkv;",
     [TA.test_attention_against_exact_f64, TA.test_attention_window_heads_and_ring_invariance]),
    ("attention reads the ring at the position, not its slot",
     "sc[p - lo] = orc_dot_q8_0(kc + ((p % cap) * nkv + g) * row, qh, hd);",
     "sc[p - lo] = orc_dot_q8_0(kc + ((p % (cap + 1) % cap) * nkv + g) * row, qh, hd);",
     [TA.test_attention_against_exact_f64]),
]


def _build(tmp, src_text):
    d = os.path.join(tmp, "src")
    os.makedirs(d, exist_ok=True)
    shutil.copy(os.path.join(ORACLE, "moe_oracle.h"), d)
    shutil.copy(os.path.join(ORACLE, "cpu_baseline.c"), d)
    with open(os.path.join(d, "moe_oracle.c"), "w") as f:
        f.write(src_text)
    lib = os.path.join(tmp, "libmut.so")
    subprocess.run(["gcc", "-O2", "-std=gnu11", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared",
                    os.path.join(d, "moe_oracle.c"), os.path.join(d, "cpu_baseline.c"), "-lm", "-lpthread",
                    "-o", lib], check=True)
    return lib


@pytest.fixture
def swap_oracle():
    """Yields a function that points the oracle module at another library; restores it after."""
    saved = O._lib

    def use(path):
        L = C.CDLL(path)
        O._declare(L)
        O._lib = L
        return O

    yield use
    O._lib = saved


def test_unmutated_copy_passes_every_pinning_test(tmp_path, swap_oracle):
    src = open(os.path.join(ORACLE, "moe_oracle.c")).read()
    orc = swap_oracle(_build(str(tmp_path), src))
    for _, _, _, tests in MUTATIONS:
        for t in tests:
            t(orc)


@pytest.mark.parametrize("name,old,new,tests", MUTATIONS, ids=[m[0] for m in MUTATIONS])
def test_planted_mistake_is_caught(tmp_path, swap_oracle, name, old, new, tests):
    src = open(os.path.join(ORACLE, "moe_oracle.c")).read()
    assert src.count(old) == 1, f"planting site for '{name}' not found exactly once"
    orc = swap_oracle(_build(str(tmp_path), src.replace(old, new)))
    for t in tests:
        with pytest.raises(AssertionError):
            t(orc)
