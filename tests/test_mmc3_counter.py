"""The MMC3 scanline counter in closed form (ghostrun-lab_amd/csrc/nes_dev.h mmc3_after_clocks, mmc3_clocks_upto),
which the device applies to a whole span of clocks at once, against the per-clock rule the oracle applies at every
clock dot (oracle/nes_oracle.c, patch:1881-1903): compiled from the product header with hipcc and run on the host,
over every counter, reload flag and latch and up to two frames of clocks, and the clock dots of a frame against a
walk over every dot."""
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HIPCC = '/opt/rocm/bin/hipcc'

PROGRAM = r'''
#include "nes_dev.h"
#include <cstdio>
int main() {
    long bad = 0, runs = 0;
    for (uint32_t cnt = 0; cnt < 256; ++cnt)
        for (uint32_t reload = 0; reload < 2; ++reload)
            for (uint32_t latch = 0; latch < 256; ++latch) {
                uint32_t c = cnt, rl = reload;
                bool any_zero = false;
                for (uint32_t n = 1; n <= 520; ++n) {
                    if (c == 0 || rl) { c = latch; rl = 0; } else { --c; }   // one clock
                    any_zero = any_zero || c == 0;
                    bool zero = false;
                    const uint32_t got = nd::mmc3_after_clocks(cnt, reload, latch, n, &zero);
                    bad += got != c || zero != any_zero;
                    ++runs;
                }
            }
    // clock dots of a frame: lines 0-239 at dot 266, the pre-render line 261 at dot 256
    uint32_t count = 0;
    for (uint32_t x = 0; x < NES_FRAME_DOTS; ++x) {
        const uint32_t line = x / 341, d = x % 341;
        if ((line < 240 && d == 266) || (line == 261 && d == 256)) ++count;
        bad += nd::mmc3_clocks_upto(x) != count;
        ++runs;
    }
    std::printf("%ld %ld %u\n", runs, bad, count);
    return 0;
}
'''


@pytest.mark.skipif(not Path(HIPCC).exists(), reason='hipcc not installed')
def test_closed_form_counter_equals_clocking_one_at_a_time(tmp_path):
    src = tmp_path / 'mmc3_check.hip'
    src.write_text(PROGRAM)
    exe = tmp_path / 'mmc3_check'
    subprocess.run([HIPCC, '-O2', '-std=c++17', '--offload-arch=gfx950', f'-I{ROOT / "include"}',
                    f'-I{ROOT / "ghostrun-lab_amd" / "csrc"}', str(src), '-o', str(exe)], check=True,
                   capture_output=True)
    runs, bad, clocks = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    assert int(runs) == 256 * 2 * 256 * 520 + 341 * 262 and int(bad) == 0 and int(clocks) == 241, (runs, bad, clocks)
