// CPU check of the persistent step's abort-word handling (fast-dllm-relax_amd/csrc/step_status.hpp),
// compiled and run by tests/test_step_status.py.  Prints "ok" or the first failed expectation.
#include <cstdio>

#include "step_status.hpp"

using fdllm::step_check_default;
using fdllm::take_step_abort;

static int fails = 0;
#define EXPECT(cond)                                          \
  do {                                                        \
    if (!(cond)) {                                            \
      std::printf("failed: %s (line %d)\n", #cond, __LINE__); \
      ++fails;                                                \
    }                                                         \
  } while (0)

int main() {
  // a clear word: nothing reported, the persistent path stays on
  volatile unsigned word = 0u;
  bool on = true;
  EXPECT(!take_step_abort(&word, &on));
  EXPECT(on);
  // a set word (an aborted launch): reported once, cleared, the path turned off
  word = 1u;
  EXPECT(take_step_abort(&word, &on));
  EXPECT(word == 0u);
  EXPECT(!on);
  EXPECT(!take_step_abort(&word, &on));  // the next entry point sees nothing more
  // any nonzero value counts; a null flag pointer is allowed
  word = 7u;
  EXPECT(take_step_abort(&word, nullptr));
  EXPECT(word == 0u);
  // no word at all (persistent path never set up)
  EXPECT(!take_step_abort(nullptr, &on));
  // the launching call checks by default whenever the persistent path is on
  EXPECT(step_check_default(true, nullptr));
  EXPECT(!step_check_default(false, nullptr));
  EXPECT(!step_check_default(true, "0"));
  EXPECT(step_check_default(false, "1"));
  EXPECT(step_check_default(true, ""));
  if (fails == 0) std::printf("ok\n");
  return fails == 0 ? 0 : 1;
}
