"""CPU bounds check of the index math of the forward kernels' tails.

The output transforms that run inside the decode-matvec kernels read and
write tagged 64-bit slots in the workspace and take dummy loads for absent
operands.  The kernels form every such index with the functions of
quipsharp_amd/csrc/qs_slots.h, and the workspace layout sizes the regions with
the same file's slot counts; this test compiles that header with g++ into a
small checker that enumerates each index the kernels form, under the kernels'
own guards and over their thread layout (16 waves of 64 lanes, chunk
c = w + 16 u, element t = lane + 64 j), for every shape they accept, and
checks it against the size of the region it addresses.  An edit of a formula
in the header reaches the kernels and this check alike; a plausible slip (a
dropped guard, B where the region holds 2 rows, a stride of m + 256) fails.

Guards and loops followed (qs_forward_dev.h, qs_linear_fused.hip,
qs_linear_batched.hip, qs_linear_big.hip):
  poll_load / load_partials_raw: c < S_m, g < SG, b < B
  reduction stores (both decode loops): row blocks rb < m / 16, rows < 16
  store_h2 (level 1): c < S_m, b < B (B <= 2)
  poll_columns (level 2): v = tid + 1024 k, (c, tt) = (v / 16, v % 16), c < S_m
  output stage and dummy loads: r < S_m, t < 256 (su words: that / 32)
"""
import shutil
import subprocess
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parents[1] / "quipsharp_amd" / "csrc"

CHECKER = r"""
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>
#include "qs_slots.h"
using namespace qs;

static int fails = 0;
static void check(size_t idx, size_t cap, const char* what, int S, int B, int SG) {
  if (idx >= cap) {
    if (fails < 5) std::printf("OUT %s: index %zu outside %zu (S %d B %d SG %d)\n", what, idx, cap, S, B, SG);
    ++fails;
  }
}

// every slot a tail polls (poll_load / load_partials_raw); unguarded: the
// planted slip without c < S_m
static void polls(int S, int B, int SG, size_t cap, const char* what, bool unguarded) {
  const int m = 256 * S, cpw = (S + 15) / 16;
  for (int g = 0; g < SG; ++g)
    for (int b = 0; b < B; ++b)
      for (int w = 0; w < 16; ++w)
        for (int u = 0; u < cpw + (unguarded ? 1 : 0); ++u) {
          const int c = w + 16 * u;
          if (!unguarded && c >= S) continue;
          for (int lane = 0; lane < 64; ++lane)
            for (int j = 0; j < 4; ++j) check(partial_index(g, B, b, m, chunk_elem(c, lane, j)), cap, what, S, B, SG);
        }
}

// the reduction stores: each slot written once
static void reductions(int S, int B, int SG, size_t cap) {
  const int m = 256 * S;
  std::vector<unsigned char> seen(cap, 0);
  for (int sg = 0; sg < SG; ++sg)
    for (int bc = 0; bc < B; ++bc)
      for (int rb = 0; rb < m / 16; ++rb)
        for (int row = 0; row < 16; ++row) {
          const size_t i = partial_index(sg, B, bc, m, block_elem(rb, row));
          check(i, cap, "reduction store", S, B, SG);
          if (i < cap) {
            if (seen[i]) { std::printf("TWICE reduction store %zu\n", i); ++fails; }
            seen[i] = 1;
          }
        }
  for (size_t i = 0; i < cap; ++i)
    if (!seen[i]) { std::printf("UNWRITTEN slot %zu (S %d B %d SG %d)\n", i, S, B, SG); ++fails; break; }
}

// level 1 (store_h2) and level 2 (poll_columns) of the two-level transform
static void two_level(int S, int B) {
  const int m = 256 * S;
  const size_t cap = h2_slot_count(m);
  for (int b = 0; b < B; ++b) {
    for (int c = 0; c < S; ++c)
      for (int lane = 0; lane < 64; ++lane)
        for (int j = 0; j < 4; ++j) check(h2_index(b, m, chunk_elem(c, lane, j)), cap, "store_h2", S, B, 0);
    for (int g = 0; g < 16; ++g)
      for (int tid = 0; tid < 1024; ++tid)
        for (int k = 0; k < 2; ++k) {
          const int v = tid + 1024 * k, c = v >> 4, tt = v & 15;
          if (c < S) check(h2_index(b, m, column_elem(c, g, tt)), cap, "poll_columns", S, B, 0);
        }
  }
}

// output stage: outputs, su (values or sign-bit words), bias, and the
// dummy loads that stand in for an absent bias (from >= 2 m slots)
static void outputs(int S) {
  const int m = 256 * S;
  for (int r = 0; r < S; ++r)
    for (int t = 0; t < 256; ++t) {
      const int o = out_elem(r, t);
      check(o, m, "output / bias / su", S, 0, 0);
      check(o >> 5, (m + 31) / 32, "su sign-bit words", S, 0, 0);
      check(o, h2_slot_count(m), "dummy load from the slots", S, 0, 0);
    }
}

int main(int argc, char** argv) {
  const char* mode = argc > 1 ? argv[1] : "";
  if (!std::strcmp(mode, "batched")) {        // the 16-row decode-matvec's tail
    for (int S : {1, 2, 3, 7, 16, 20, 43, 48})
      for (int B : {3, 8, 15, 16})
        for (int SG : {1, 2, 3, 7}) {
          const size_t cap = batched_slot_count(SG, B, 256 * S);
          polls(S, B, SG, cap, "poll", false);
          reductions(S, B, SG, cap);
        }
  } else if (!std::strcmp(mode, "one_launch")) {  // the one-launch kernel (1-2 rows)
    for (int S : {1, 4, 16, 20, 43, 64, 100, 128})
      for (int B : {1, 2})
        for (int SG : {1, 2, 5, 8}) {
          if (S <= 16) polls(S, B, SG, fused_slot_count(SG, 256 * S), "one-launch poll", false);
          else two_level(S, B);
          reductions(S, B, SG, fused_slot_count(SG, 256 * S) / 2 * B);
        }
  } else if (!std::strcmp(mode, "outputs")) {
    for (int S : {1, 16, 43, 48, 100, 128}) outputs(S);
  } else if (!std::strcmp(mode, "slip")) {     // a poll without its c < S_m guard
    polls(20, 16, 2, batched_slot_count(2, 16, 256 * 20), "unguarded poll", true);
  } else {
    std::printf("usage: checker batched|one_launch|outputs|slip\n");
    return 2;
  }
  std::printf("fails %d\n", fails);
  return fails ? 1 : 0;
}
"""


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    d = tmp_path_factory.mktemp("tailbounds")
    (d / "checker.cpp").write_text(CHECKER)
    exe = d / "checker"
    subprocess.run([gxx, "-O2", "-std=c++17", "-Wall", "-I", str(CSRC), str(d / "checker.cpp"), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    return exe


def _run(exe, mode):
    return subprocess.run([str(exe), mode], capture_output=True, text=True, timeout=300)


@pytest.mark.parametrize("mode", ["batched", "one_launch", "outputs"])
def test_tail_indices_in_bounds(checker, mode):
    r = _run(checker, mode)
    assert r.returncode == 0 and "fails 0" in r.stdout, r.stdout + r.stderr


def test_a_planted_slip_is_caught(checker):
    """A poll that skipped its c < S_m guard would read past the region."""
    r = _run(checker, "slip")
    assert r.returncode == 1 and "OUT unguarded poll" in r.stdout, r.stdout + r.stderr
