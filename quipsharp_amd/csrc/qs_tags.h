// Launch tags of the tagged partial-sum slots (64-bit {fp32 value, tag}),
// shared by the forward kernels (qs_forward_dev.h) and host-side checks
// compiled without HIP (a plain C++ compiler sees the same functions).
//
// A tag is a quiet-NaN bit pattern (an fp32 NaN, and an fp16 NaN in its upper
// half) holding a 20-bit launch counter c (1 .. 2^20 - 1) in bits 2-21 and the
// job's index g (0-3) in bits 0-1.  The workspace's first 256 bytes hold, per
// job index g, the epoch word (unsigned word g: the tag of the last launch,
// zero before the first) and the wrap word (unsigned word kWrapWord + g).
#pragma once

#include <stddef.h>
#include <stdint.h>

#if defined(__HIPCC__) || defined(__HIP__)
#define QS_HD __host__ __device__
#else
#define QS_HD
#endif

namespace qs {

constexpr uint32_t kTagBase = 0x7FC00000u;
constexpr uint32_t kTagJobMask = 0xFFC00003u;  // the NaN base and the job index
constexpr uint32_t kTagCounterMax = 0xFFFFFu;  // the last counter value before it starts again at 1
constexpr int kWrapWord = 16;                  // unsigned index of job 0's wrap word
constexpr int kWsHeaderWords = 32;             // 64-bit words of the header (256 bytes)

QS_HD inline uint32_t tag_counter(uint32_t tag) { return (tag >> 2) & kTagCounterMax; }

// The tag of the launch after the one whose tag is `epoch` (zero: none yet).
QS_HD inline uint32_t next_tag(uint32_t epoch, int g) {
  const uint32_t c = (tag_counter(epoch) + 1u) & kTagCounterMax;
  return kTagBase | ((c ? c : 1u) << 2) | (uint32_t)g;
}

// Counter wrap.  Slot positions depend on m, n and the batch rows, so a slot
// that a launch wrote and no later launch has overwritten keeps that launch's
// tag; once the counter comes back to the same value, 2^20 - 1 launches of
// job index g later, the slot would pass for one of the new launch.  So the
// launch with the last counter value (wrap_launch) removes every tag of job
// index g from the workspace before the counter starts again: its tail
// work-groups count themselves in the job's wrap word once they have read
// every slot they poll, and the last of them overwrites with zero each 64-bit
// word past the header whose high word is a tag of job index g
// (slot_of_job).  The launch before it (wrap_reset_launch) sets the wrap word
// to zero, so the count starts from zero whatever the word held.
QS_HD inline bool wrap_launch(uint32_t tag) { return tag_counter(tag) == kTagCounterMax; }
QS_HD inline bool wrap_reset_launch(uint32_t tag) { return tag_counter(tag) == kTagCounterMax - 1u; }
QS_HD inline bool slot_of_job(unsigned long long word, int g) {
  return ((uint32_t)(word >> 32) & kTagJobMask) == (kTagBase | (uint32_t)g);
}

// Where a tagged launch finds its workspace: the job's wrap word, the
// workspace and its size (the wrap clear scans it), and how many tail
// work-groups the job has (each counts itself once in a wrap launch).
struct TagWs {
  unsigned* wrap;
  unsigned long long* base;
  unsigned long long words;
  int ntail;
};

// TagWs of job index g in the workspace ws of `bytes` bytes (ntail is the
// launcher's).
inline TagWs tag_ws(void* ws, size_t bytes, int g) {
  TagWs t;
  t.wrap = static_cast<unsigned*>(ws) + kWrapWord + g;
  t.base = static_cast<unsigned long long*>(ws);
  t.words = bytes / 8;
  t.ntail = 0;
  return t;
}

}  // namespace qs
