"""The teaching trainer's host logic on the CPU: the oracle pinned against the C++ standard and libstdc++, and the
library's own draw, schedule, chunk checks, chunk choice and command-line errors against the oracle (none of these
touch the GPU)."""
from __future__ import annotations

import ctypes
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

from flyguy_amd._lib import lib
from oracle import trainer as ot

cll = ctypes.c_longlong


def test_mt19937_64_known_answer():
    # [rand.predef]: the 10000th consecutive invocation of a default-constructed mt19937_64 yields 9981545732273789042
    g = ot.MT19937_64()
    for _ in range(9999):
        g()
    assert g() == 9981545732273789042


PROBE = r"""
#include <cstdio>
#include <random>
int main() {
    const long long totals[] = {1, 2, 3, 1000, 1099511627783LL, 6917529027641081856LL, 9223372036854775807LL};
    const unsigned long long seeds[] = {12345ULL, 4242ULL, 99991ULL * 7 + 3};
    for (unsigned long long seed : seeds) {
        std::mt19937_64 raw(seed);
        for (int i = 0; i < 3; ++i) printf("raw %llu %llu\n", seed, (unsigned long long)raw());
        for (long long total : totals) {
            std::mt19937_64 r(seed);
            std::uniform_int_distribution<long long> u(0, total - 1);
            for (int i = 0; i < 40; ++i) printf("u %llu %lld %lld\n", seed, total, u(r));
        }
    }
    return 0;
}
"""


@pytest.fixture(scope="module")
def libstdcxx_draws(tmp_path_factory):
    gxx = shutil.which("g++")
    if not gxx:
        pytest.skip("g++ not available")
    d = tmp_path_factory.mktemp("probe")
    (d / "p.cpp").write_text(PROBE)
    subprocess.run([gxx, "-O1", "-std=c++17", str(d / "p.cpp"), "-o", str(d / "p")], check=True)
    return subprocess.run([str(d / "p")], check=True, capture_output=True, text=True).stdout.splitlines()


def test_oracle_matches_libstdcxx(libstdcxx_draws):
    raw = {}
    uni = {}
    for line in libstdcxx_draws:
        f = line.split()
        if f[0] == "raw":
            raw.setdefault(int(f[1]), []).append(int(f[2]))
        else:
            uni.setdefault((int(f[1]), int(f[2])), []).append(int(f[3]))
    for seed, want in raw.items():
        g = ot.MT19937_64(seed)
        assert [g() for _ in want] == want
    rejections = 0
    for (seed, total), want in uni.items():
        g = ot.MT19937_64(seed)
        got = [ot.uniform(g, 0, total - 1) for _ in want]
        assert got == want, (seed, total)
        rejections += int(g.i != len(want))     # engine calls beyond one per draw: the rejection branch ran
    assert rejections > 0


def _ft_draw(seed, sizes, B, nb):
    out = np.zeros((nb * B, 2), np.int32)
    s = (cll * len(sizes))(*sizes)
    assert lib().ft_draw(seed, s, len(sizes), B, nb, out.ctypes.data) == 0
    return out


@pytest.mark.parametrize("sizes", [[1], [7], [3, 1, 4], [100, 0, 250, 9], [2 ** 31 - 1, 5]])
def test_draw_matches_oracle(sizes):
    for seed in (12345, 12345 + 7, 1000003 * 11 + 7):
        got = _ft_draw(seed, sizes, 32, 3)
        want = ot.draws(seed, sizes, 32, 3)
        assert np.array_equal(got, want), (seed, sizes)
        for c, smp in got:
            assert 0 <= smp < sizes[c]


def test_draw_rejects_bad_sizes():
    s = (cll * 2)(0, 0)
    out = np.zeros(64, np.int32)
    assert lib().ft_draw(1, s, 2, 32, 1, out.ctypes.data) == -1
    s = (cll * 1)(-3)
    assert lib().ft_draw(1, s, 1, 32, 1, out.ctypes.data) == -1


def _ft_lr(step, *a):
    out = (ctypes.c_float * 3)()
    lib().ft_lr(step, *a, out)
    return np.array(out[:], np.float32)


def test_lr_schedule():
    args = (3e-4, 1e-4, 3e-4, 3e-5, 20000.0)
    for step in (0, 1, 2, 999, 20000, 40000, 66438, 66439, 10 ** 6, 10 ** 9):
        got = _ft_lr(step, *args)
        assert np.array_equal(got, ot.lr(step, *args)), step
    # closed forms: the base rate at step 0, half of it one half-life later, the floor lr_min * base / lr far away
    assert np.array_equal(_ft_lr(0, *args), np.float32([3e-4, 1e-4, 3e-4]))
    assert np.allclose(_ft_lr(20000, *args), np.float32([1.5e-4, 0.5e-4, 1.5e-4]), rtol=1e-6)
    assert np.allclose(_ft_lr(10 ** 7, *args), np.float32([3e-5, 1e-5, 3e-5]), rtol=1e-6)


def test_chunk_checks(tmp_path):
    rng = np.random.default_rng(0)
    good = tmp_path / "chunk_0000.bin"
    ot.write_chunk(good, rng.standard_normal((11, 5)), rng.standard_normal((11, 3)))
    cases = {"good": good}
    raw = good.read_bytes()
    for name, data in {"magic": b"FLYX" + raw[4:], "short": raw[:-1], "zero": b"FLYD" + struct.pack("<qii", 0, 5, 3),
                       "empty": b""}.items():
        p = tmp_path / f"chunk_{name}.bin"
        p.write_bytes(data)
        cases[name] = p
    for name, p in cases.items():
        for od, na in ((5, 3), (5, 4), (6, 3)):
            got = lib().ft_chunk_samples(str(p).encode(), od, na)
            assert got == ot.chunk_samples(p, od, na), (name, od, na)
    assert lib().ft_chunk_samples(str(good).encode(), 5, 3) == 11
    assert lib().ft_chunk_samples(str(tmp_path / "missing.bin").encode(), 5, 3) == -1


def test_scan_order(tmp_path):
    names = ["chunk_0003.bin", "chunk_0001.bin", "chunk_0002.bin", "chunk_0000.bin", "chunk_x.tmp", "other.bin",
             "chunk_0004.bin"]
    t0 = 1_700_000_000 * 10 ** 9
    for i, n in enumerate(names):
        (tmp_path / n).write_bytes(b"x")
        # chunk_0000 and chunk_0004 share a time stamp: the path breaks the tie
        ns = t0 + (3 if n == "chunk_0004.bin" else i) * 10 ** 9
        os.utime(tmp_path / n, ns=(ns, ns))
    buf = ctypes.create_string_buffer(4096)
    for keep in (0, 1, 2, 3, 10):
        n = lib().ft_scan_order(str(tmp_path).encode(), keep, buf, 4096)
        got = buf.value.decode().split("\n") if n else []
        want = ot.scan_order(tmp_path, keep)
        assert got == want and n == len(want), keep
    assert ot.scan_order(tmp_path, 10) == ["chunk_0003.bin", "chunk_0001.bin", "chunk_0002.bin", "chunk_0000.bin",
                                           "chunk_0004.bin"]
    assert lib().ft_scan_order(str(tmp_path).encode(), 10, buf, 8) == -1        # does not fit


def _main(*args):
    argv = (ctypes.c_char_p * (len(args) + 1))(b"flyguy_train", *[a.encode() for a in args])
    return lib().ft_main(len(args) + 1, argv)


def test_command_line_errors(capfd):
    assert _main() == 2
    assert "usage: flyguy_train" in capfd.readouterr().err
    assert _main("NET", "P", "D", "O", "--bogus", "1") == 2
    assert "unknown option --bogus" in capfd.readouterr().err
    assert _main("NET", "P", "D", "O", "--batch", "33") == 2
    assert "--batch must be a multiple of 32" in capfd.readouterr().err


def test_executable_usage():
    exe = lib()._name.replace("libflyguy_core.so", "flyguy_train")
    r = subprocess.run([exe], capture_output=True, text=True)
    assert r.returncode == 2 and "usage: flyguy_train" in r.stderr
