// Host side of the persistent cached step's abort word (host code only; no HIP dependency).
//
// The opt-in persistent step (step_body.hpp) bounds every grid-barrier wait by a wall-clock deadline; a
// workgroup that times out sets an abort word in pinned host memory, every workgroup leaves, and the
// launch's hidden states and cache rows are invalid.  Each entry point that consumes or extends a step's
// results first takes the word: a set word is reported once (the entry point then fails with an error
// instead of returning results computed from the aborted launch), cleared, and the persistent path is
// turned off for the rest of the context's life, so the per-operator kernels serve every later call.
#pragma once

namespace fdllm {

// true (once) when the word is set; clears it and turns the persistent path off
inline bool take_step_abort(volatile unsigned* word, bool* step_on) {
  if (word == nullptr || *word == 0u) return false;
  *word = 0u;
  if (step_on != nullptr) *step_on = false;
  return true;
}

// Whether every persistent launch is waited for and its word checked by the call that launched it:
// on unless FDLLM_STEP_CHECK says otherwise (env_value null: not set).  Without the check an aborted
// launch is reported by the next entry point that takes the word.
inline bool step_check_default(bool persistent_on, const char* env_value) {
  if (env_value != nullptr && env_value[0] != '\0') return env_value[0] != '0';
  return persistent_on;
}

}  // namespace fdllm
