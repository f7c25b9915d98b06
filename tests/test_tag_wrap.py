"""CPU check of the launch tags of the tagged partial-sum slots and of the
counter wrap (quipsharp_amd/csrc/qs_tags.h, compiled here with g++: the
same functions the kernels call).

The simulation follows the kernels' protocol on a small workspace: a launch
of job index g reads the epoch word, takes next_tag, its producers write
tagged slots at positions that depend on the batch rows (B = 2 reaches
slots that B = 1 never writes, as y1t + (g B + b) m does), and its tail
work-groups end as finish_tagged_launch does (epoch store, wrap word reset
one launch before the wrap, count and clear on the wrap launch).  A slot
that already carries the tag of a launch before its producers write is the
hazard a polling tail could take for fresh.  With the clear switched off
the scenario must produce that hazard once the counter comes round; with it,
never."""
import shutil
import subprocess
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parents[1] / "quipsharp_amd" / "csrc"

SIM = r"""
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>
#include "qs_tags.h"
using namespace qs;

static unsigned long long tagged(float v, uint32_t tag) {
  uint32_t u; std::memcpy(&u, &v, 4);
  return ((unsigned long long)tag << 32) | u;
}

struct Ws {
  std::vector<unsigned long long> w;
  explicit Ws(size_t words) : w(words, 0ull) {}
  uint32_t* u32() { return reinterpret_cast<uint32_t*>(w.data()); }
};

static long hazards = 0, clears = 0;

// one launch of job index g with B rows: K slots per row from word `base`
static void launch(Ws& ws, int g, int B, int K, size_t base, bool clear_on) {
  const uint32_t tag = next_tag(ws.u32()[g], g);
  for (size_t p = base; p < base + (size_t)B * K; ++p)
    if ((uint32_t)(ws.w[p] >> 32) == tag) ++hazards;       // a poll before the write would accept it
  for (size_t p = base; p < base + (size_t)B * K; ++p) ws.w[p] = tagged(1.0f, tag);
  TagWs t = tag_ws(ws.w.data(), ws.w.size() * 8, g);
  t.ntail = B;
  for (int tail = 0; tail < t.ntail; ++tail) {             // finish_tagged_launch of each tail work-group
    ws.u32()[g] = tag;
    if (wrap_reset_launch(tag)) *t.wrap = 0;
    if (!wrap_launch(tag) || !clear_on) continue;
    const unsigned done = ++*t.wrap;
    if (done != (unsigned)t.ntail) continue;
    *t.wrap = 0;
    ++clears;
    for (unsigned long long i = kWsHeaderWords; i < t.words; ++i)
      if (slot_of_job(t.base[i], g)) t.base[i] = 0ull;
  }
}

int main(int argc, char** argv) {
  const bool clear_on = argc > 1 && std::atoi(argv[1]) != 0;
  // tag format
  for (int g = 0; g < 4; ++g) {
    uint32_t e = 0;
    for (uint32_t c = 1; c <= kTagCounterMax + 3; ++c) {
      const uint32_t t = next_tag(e, g);
      const uint32_t want = c <= kTagCounterMax ? c : c - kTagCounterMax;  // 0 is skipped
      if (tag_counter(t) != want || (int)(t & 3u) != g) { std::printf("FAIL counter %u g %d\n", c, g); return 1; }
      float f; std::memcpy(&f, &t, 4);
      const uint32_t hi16 = t >> 16;
      if (!std::isnan(f) || (hi16 & 0x7C00u) != 0x7C00u || (hi16 & 0x3FFu) == 0) { std::printf("FAIL nan %08x\n", t); return 1; }
      for (int h = 0; h < 4; ++h)
        if (slot_of_job(tagged(0.5f, t), h) != (h == g)) { std::printf("FAIL job %08x %d\n", t, h); return 1; }
      if (wrap_launch(t) != (tag_counter(t) == kTagCounterMax)) { std::printf("FAIL wrap\n"); return 1; }
      e = t;
    }
  }
  if (slot_of_job(0ull, 0) || slot_of_job(tagged(1.0f, 0u), 0)) { std::printf("FAIL zero slot\n"); return 1; }
  // scenario: job 0 mostly at 1 row, one 2-row launch early on; the 2-row
  // slots past the first row are left behind until the counter returns to
  // that launch's value; job 1 runs beside it and must keep its slots
  Ws ws(4096);
  ws.u32()[kWrapWord] = 12345u;                            // whatever the wrap word held
  const int K = 256;
  const size_t base = kWsHeaderWords;
  launch(ws, 0, 1, K, base, clear_on);
  launch(ws, 0, 2, K, base, clear_on);                     // counter 2: slots base + K .. base + 2K
  for (uint32_t i = 0; i < kTagCounterMax - 3; ++i) launch(ws, 0, 1, K, base, clear_on);  // counters 3 .. 2^20 - 2
  // job 1 in its own region, its slots written just before job 0 wraps
  for (int i = 0; i < 3; ++i) launch(ws, 1, 2, K, base + 2048, clear_on);
  const unsigned long long job1 = ws.w[base + 2048];
  launch(ws, 0, 1, K, base, clear_on);                     // counter 2^20 - 1: the wrap launch
  if (clear_on && ws.w[base + 2048] != job1) { std::printf("FAIL job 1 slots cleared\n"); return 1; }
  launch(ws, 0, 1, K, base, clear_on);                     // counter 1
  launch(ws, 0, 2, K, base, clear_on);                     // counter 2 again, 2 rows
  std::printf("tag_counter %u hazards %ld clears %ld wrap %u\n", tag_counter(ws.u32()[0]), hazards, clears,
              ws.u32()[kWrapWord]);
  return 0;
}
"""


@pytest.fixture(scope="module")
def sim(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    d = tmp_path_factory.mktemp("tagwrap")
    (d / "sim.cpp").write_text(SIM)
    exe = d / "sim"
    subprocess.run([gxx, "-O2", "-std=c++17", "-Wall", "-I", str(CSRC), str(d / "sim.cpp"), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    return exe


def _run(exe, clear_on):
    r = subprocess.run([str(exe), "1" if clear_on else "0"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    out = dict(zip(*[iter(r.stdout.split())] * 2))
    return {k: int(v) for k, v in out.items()}


def test_stale_slot_returns_without_the_wrap_clear(sim):
    """The scenario has teeth: without the clear, the 2-row launch at counter
    2 after the wrap finds slots of the 2-row launch at counter 2 before it."""
    r = _run(sim, False)
    assert r["tag_counter"] == 2 and r["hazards"] > 0 and r["clears"] == 0


def test_wrap_clear_removes_stale_slots(sim):
    r = _run(sim, True)
    assert r["tag_counter"] == 2
    assert r["clears"] == 1, r      # exactly the wrap launch's last tail work-group
    assert r["hazards"] == 0, r
    assert r["wrap"] == 0, r        # the wrap word is back at zero
