"""Pins Philox4x32 (oracle and the library's host build): ten rounds by the Random123
known-answer vectors and by rocRAND's philox4x32_10; any round count, the stochastic-rounding
stream's seven included, by rocRAND's own round and key-bump functions."""
import os
import shutil
import subprocess

import numpy as np
import pytest

import mdq_hip
from oracle import mdq_oracle as orc

KAT = [  # (counter, key, output) from the Random123 distribution's kat_vectors
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,out", KAT)
def test_philox_kat(ctr, key, out):
    assert tuple(int(v) for v in orc.philox4x32_10(ctr, key)) == out
    assert tuple(int(v) for v in mdq_hip.host_philox(ctr, key)) == out


PROBE = r'''
#include <cstdio>
#include <cstdlib>
#include <hip/hip_runtime.h>
// rocRAND's round and key-bump functions are private members of its engine; the probe opens
// them to apply the published round function any number of times
#define private public
#include <rocrand/rocrand_philox4x32_10.h>
#undef private
struct probe : rocrand_device::philox4x32_10_engine {
  uint4 run(uint4 c, uint2 k) { return ten_rounds(c, k); }
  // R rounds from rocRAND's own round and key schedule
  static uint4 rounds(uint4 c, uint2 k, int R) {
    for (int r = 0; r < R; ++r) { if (r) k = bumpkey(k); c = single_round(c, k); }
    return c;
  }
};
int main() {
  probe e; unsigned a[7];
  while (scanf("%x %x %x %x %x %x %x", a, a+1, a+2, a+3, a+4, a+5, a+6) == 7) {
    uint4 c{a[0], a[1], a[2], a[3]};
    uint2 k{a[4], a[5]};
    uint4 r = a[6] == 10 ? e.run(c, k) : probe::rounds(c, k, (int)a[6]);
    printf("%x %x %x %x\n", r.x, r.y, r.z, r.w);
  }
}
'''


@pytest.mark.skipif(not os.path.exists("/opt/rocm/include/rocrand/rocrand_philox4x32_10.h")
                    or shutil.which("hipcc") is None, reason="rocRAND headers / hipcc absent")
def test_philox_matches_rocrand(tmp_path):
    src = tmp_path / "probe.cpp"
    src.write_text(PROBE)
    exe = tmp_path / "probe"
    subprocess.run(["hipcc", "-O1", "--offload-arch=gfx950", str(src), "-o", str(exe)], check=True,
                   capture_output=True, timeout=300)
    rng = np.random.default_rng(3)
    rows = rng.integers(0, 2**32, size=(300, 6), dtype=np.uint64)
    rounds = [10, orc.SR_ROUNDS, 1, 2, 5]
    jobs = [(r, R) for R in rounds for r in rows[:300 if R in (10, orc.SR_ROUNDS) else 20]]
    inp = "\n".join(" ".join(f"{int(v):x}" for v in r) + f" {R:x}" for r, R in jobs) + "\n"
    out = subprocess.run([str(exe)], input=inp, capture_output=True, text=True, check=True).stdout.split("\n")
    for (r, R), line in zip(jobs, out):
        want = [int(x, 16) for x in line.split()]
        got = orc.philox4x32_10(r[:4], r[4:]) if R == 10 else orc.philox4x32(r[:4], r[4:], R)
        assert [int(v) for v in got] == want, R
        assert [int(v) for v in orc.philox4x32(r[:4], r[4:], R)] == want, R
