"""The address-word helper of the kernels (``monarch_muon_amd/csrc/addr.hpp``),
compiled for the host with g++: a 64-bit address split into two 32-bit words
and joined again is the same address for every low word, bit 31 set or not;
the same join with the low word taken as a signed ``int`` (what a
readfirstlane builtin returns) corrupts exactly the addresses whose low word
has bit 31 set, the failure the helper exists to prevent."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent

PROG = r'''
#include <stdio.h>
#include "addr.hpp"
using namespace mmuon;
int main() {
  const unsigned long long cases[] = {0x00007f3a80001000ull, 0x00007f3a7ffff000ull, 0x0000000080000000ull,
                                      0x00007fffffffffffull, 0x000055d0c0de0010ull, 0x0000000000000000ull};
  for (unsigned long long a : cases) {
    const int slo = int(low_word(a)), shi = int(high_word(a));   // as readfirstlane returns them
    const unsigned long long good = join_words(uint32_t(slo), uint32_t(shi));
    const unsigned long long bad = (static_cast<unsigned long long>(shi) << 32) | static_cast<long long>(slo);
    printf("%016llx %016llx %016llx\n", a, good, bad);
  }
  return 0;
}
'''


def test_join_words_round_trips_every_low_word(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    src, exe = tmp_path / "t.cpp", tmp_path / "t"
    src.write_text(PROG)
    subprocess.run([gxx, "-std=c++17", "-O2", f"-I{ROOT / 'monarch_muon_amd' / 'csrc'}", str(src), "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    rows = [tuple(int(w, 16) for w in line.split()) for line in out if line.strip()]
    assert len(rows) == 6
    for a, good, bad in rows:
        assert good == a
        if a & 0x80000000:
            assert bad == (a | 0xFFFFFFFF00000000)     # sign-extended: the fault this helper prevents
        else:
            assert bad == a
