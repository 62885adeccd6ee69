"""The device's tanhf (rosevine_amd/csrc/tanhf.hpp) against the host C library's tanhf.

Rust's f32::tanh, inside the reference's GELU (runtime/src/ops.rs:145-149), is the platform
tanhf. The header's restatement (fb_tanhf) and its branch-free form used by the kernels
(tanhf_select) are compiled here for the host with g++ and compared bit for bit with the host
libm over every 61st f32 bit pattern (about 70 million inputs, all ranges and both signs) plus
the boundaries of every branch. NaN results only need to be NaN on both sides.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECK = r'''
#include <cstdio>
#include <cstring>
#include "tanhf.hpp"
static uint32_t fb(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static unsigned long long bad_fb = 0, bad_sel = 0, n = 0;
static void one(uint32_t u) {
    const float x = bf(u), want = tanhf(x), a = rvm::fb_tanhf(x), b = rvm::tanhf_select(x);
    const bool wn = want != want;
    if (!(wn ? a != a : fb(a) == fb(want))) ++bad_fb;
    if (!(wn ? b != b : fb(b) == fb(want))) ++bad_sel;
    ++n;
}
int main() {
    for (unsigned long long u = 0; u <= 0xffffffffull; u += 61) one((uint32_t)u);
    const uint32_t edges[] = {0x00000000u, 0x00000001u, 0x23ffffffu, 0x24000000u, 0x3eb17218u, 0x3eb17219u,
                              0x3f3504f3u, 0x3f7fffffu, 0x3f800000u, 0x3f851592u, 0x3f851591u, 0x4195b844u,
                              0x41afffffu, 0x41b00000u, 0x7f7fffffu, 0x7f800000u, 0x7fc00000u, 0x33000000u,
                              0x32ffffffu};
    for (uint32_t e : edges)
        for (int d = -2; d <= 2; ++d) { one(e + d); one((e + d) ^ 0x80000000u); }
    printf("%llu %llu %llu\n", n, bad_fb, bad_sel);
    return 0;
}
'''


def test_device_tanhf_equals_host_libm(tmp_path):
    src = tmp_path / "check.cpp"
    src.write_text(CHECK)
    exe = tmp_path / "check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-fno-fast-math",
                    "-I", os.path.join(ROOT, "rosevine_amd", "csrc"), str(src), "-o", str(exe), "-lm"], check=True)
    n, bad_fb, bad_sel = (int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True,
                                                          check=True).stdout.split())
    assert n > 70_000_000
    assert bad_fb == 0, f"fb_tanhf differs from the host tanhf on {bad_fb} inputs"
    assert bad_sel == 0, f"tanhf_select differs from the host tanhf on {bad_sel} inputs"
