// Host side of the fault word of launches whose workgroups wait on each other (host code only; no HIP
// dependency).
//
// The one-shot projections (down, in a cached step) sum their k splits inside their own launch (GroupWait,
// kernels.hpp).  Every such wait is bounded by a wall-clock deadline; a workgroup that times
// out sets a fault word in pinned host memory and skips its share, so that launch's hidden states (and
// the calls that consumed them) are invalid.  Each entry point that consumes or extends step results
// first takes the word: a set word is reported once (the entry point then fails with an error instead of
// returning results computed after the faulted launch), cleared, and the in-launch reductions are turned
// off for the rest of the context's life, so the separate split-sum kernel serves every later
// call.
#pragma once

namespace fdllm {

// true (once) when the word is set; clears it and turns the in-launch reductions off
inline bool take_wait_fault(volatile unsigned* word, bool* waits_on) {
  if (word == nullptr || *word == 0u) return false;
  *word = 0u;
  if (waits_on != nullptr) *waits_on = false;
  return true;
}

// Whether a launch whose workgroups wait on each other may run: the switch is on, the fault word exists,
// and the grid is resident at once (at most one workgroup per compute unit, `resident` of them).
inline bool group_waits_fit(bool waits_on, const volatile unsigned* word, long long grid, long long resident) {
  return waits_on && word != nullptr && grid > 0 && grid <= resident;
}

}  // namespace fdllm
