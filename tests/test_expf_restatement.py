"""The device's expf (rosevine_amd/csrc/expf.hpp) against the host C library's expf.

Rust's f32::exp, inside the reference's softmax (runtime/src/ops.rs:170-179), is the platform
expf. The header's restatement (glibc_expf) is compiled here for the host with g++ and compared
bit for bit with the host libm over every 61st f32 bit pattern (about 70 million inputs, all
ranges and both signs), a denser pass over the softmax's range (x <= 0: every 7th negative
pattern), and the boundaries of every branch, including the one input (0xc27c65d9) where an
unfused evaluation of the same method rounds differently. NaN results only need to be NaN on
both sides. The header's table is also checked against the mathematics: entry i is the correctly
rounded double of 2^(i/32) minus i << 47.
"""
import os
import struct
import subprocess
from decimal import Decimal, getcontext

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECK = r'''
#include <cstdio>
#include <cstring>
#include "expf.hpp"
static uint32_t fb(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static unsigned long long bad = 0, n = 0;
static void one(uint32_t u) {
    const float x = bf(u), want = expf(x), got = rvm::glibc_expf(x);
    if (!(want != want ? got != got : fb(got) == fb(want))) ++bad;
    ++n;
}
int main() {
    for (unsigned long long u = 0; u <= 0xffffffffull; u += 61) one((uint32_t)u);
    for (unsigned long long u = 0x80000000ull; u <= 0xffffffffull; u += 7) one((uint32_t)u);
    const uint32_t edges[] = {0x00000000u, 0x00000001u, 0x3f800000u, 0x42b00000u, 0x42b17217u, 0x42b17218u,
                              0x42cff1b4u, 0x42ce8ecfu, 0x42cff1b5u, 0x42ce8ed0u, 0x7f7fffffu, 0x7f800000u,
                              0x7fc00000u, 0x42afffffu, 0xc27c65d9u ^ 0x80000000u};
    for (uint32_t e : edges)
        for (int d = -2; d <= 2; ++d) { one(e + d); one((e + d) ^ 0x80000000u); }
    printf("%llu %llu\n", n, bad);
    return 0;
}
'''


def test_table_is_two_to_the_i_over_32():
    getcontext().prec = 60
    ln2 = Decimal(2).ln()
    src = open(os.path.join(ROOT, "rosevine_amd", "csrc", "expf.hpp")).read()
    body = src[src.index("constexpr uint64_t T[32] = {") + len("constexpr uint64_t T[32] = {"):]
    tab = [int(v, 16) for v in body[:body.index("}")].replace("\n", " ").split(",")]
    assert len(tab) == 32
    for i, t in enumerate(tab):
        v = float((ln2 * i / 32).exp())  # correctly rounded
        assert t == struct.unpack("<Q", struct.pack("<d", v))[0] - (i << 47), i


def test_device_expf_equals_host_libm(tmp_path):
    src = tmp_path / "check.cpp"
    src.write_text(CHECK)
    exe = tmp_path / "check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-fno-fast-math",
                    "-I", os.path.join(ROOT, "rosevine_amd", "csrc"), str(src), "-o", str(exe), "-lm"], check=True)
    n, bad = (int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split())
    assert n > 370_000_000
    assert bad == 0, f"glibc_expf differs from the host expf on {bad} inputs"
