"""Host checks of csrc/bits.h, the one place where the library rebuilds a
64-bit address from two 32-bit halves.

A GPU fault was once traced to an address rebuilt from two readfirstlane
results typed int: the low half, sign-extended into the 64-bit OR, set every
upper bit whenever it was >= 2^31. compose_u64 takes both halves as uint32_t;
this test builds a host program from the header with g++ and checks it on the
halves that broke the int form, and checks that the device source rebuilds no
address any other way.
"""
import os
import re
import subprocess
import tempfile

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "custom_ops_amd", "csrc")

PROGRAM = r"""
#include <stdio.h>
#include "bits.h"
using namespace mi355fa;
int main() {
  const unsigned long long cases[] = {0x00007f1280000000ull, 0x00007fffffffffffull, 0x0000000180000010ull,
                                      0x0000000000000000ull, 0xffffffff00000001ull, 0x000055550000ffffull};
  int bad = 0;
  for (unsigned long long a : cases) {
    // the halves as readfirstlane hands them back: typed int
    const int lo_i = (int)low_u32(a), hi_i = (int)high_u32(a);
    if (compose_u64((uint32_t)lo_i, (uint32_t)hi_i) != a) bad |= 1;
    if (compose_u64(lo_i, hi_i) != a) bad |= 2;          // implicit int -> uint32_t conversion
    if (compose_u64(low_u32(a), high_u32(a)) != a) bad |= 4;
    // the form that faulted: widening the int half directly
    const unsigned long long naive = ((unsigned long long)(unsigned)hi_i << 32) | (long long)lo_i;
    if ((a & 0x80000000ull) && naive == a) bad |= 8;      // it must differ exactly when bit 31 is set
    if (!(a & 0x80000000ull) && naive != a) bad |= 16;
  }
  printf("bad=%d\n", bad);
  return bad;
}
"""


def test_compose_u64_on_the_host():
    with tempfile.TemporaryDirectory() as tmp:
        src = os.path.join(tmp, "t.cpp")
        exe = os.path.join(tmp, "t")
        with open(src, "w") as f:
            f.write(PROGRAM)
        subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", f"-I{CSRC}", src, "-o", exe], check=True,
                       timeout=120)
        res = subprocess.run([exe], capture_output=True, text=True, timeout=60)
        assert res.returncode == 0, res.stdout


def test_device_source_rebuilds_addresses_only_through_compose_u64():
    """No 64-bit value is assembled from shifted halves outside bits.h."""
    with open(os.path.join(CSRC, "fa_fwd.hip")) as f:
        src = f.read()
    code = re.sub(r"//[^\n]*", "", src)
    hits = [m.group(0) for m in re.finditer(r"<<\s*32[^;]*\|", code)]
    # the launch-tag seed mixes two random words on the host; it is no address
    hits = [h for h in hits if "rd()" not in h]
    assert not hits, hits
    assert "compose_u64(" in code
