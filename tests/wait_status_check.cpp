// CPU check of the group-wait fault word handling (fast-dllm-relax_amd/csrc/wait_status.hpp), compiled and
// run by tests/test_wait_status.py.  Prints "ok" or the first failed expectation.
#include <cstdio>

#include "wait_status.hpp"

using fdllm::group_waits_fit;
using fdllm::take_wait_fault;

static int fails = 0;
#define EXPECT(cond)                                          \
  do {                                                        \
    if (!(cond)) {                                            \
      std::printf("failed: %s (line %d)\n", #cond, __LINE__); \
      ++fails;                                                \
    }                                                         \
  } while (0)

int main() {
  // a clear word: nothing reported, the in-launch reductions stay on
  volatile unsigned word = 0u;
  bool on = true;
  EXPECT(!take_wait_fault(&word, &on));
  EXPECT(on);
  // a set word (a launch whose wait timed out): reported once, cleared, the reductions turned off
  word = 1u;
  EXPECT(take_wait_fault(&word, &on));
  EXPECT(word == 0u);
  EXPECT(!on);
  EXPECT(!take_wait_fault(&word, &on));  // the next entry point sees nothing more
  EXPECT(!on);                           // and the reductions stay off
  // any nonzero value counts; a null flag pointer is allowed
  word = 7u;
  EXPECT(take_wait_fault(&word, nullptr));
  EXPECT(word == 0u);
  // no word at all (pinned memory unavailable)
  EXPECT(!take_wait_fault(nullptr, &on));
  // a launch may wait only with the switch on, a word, and a grid that is resident at once
  EXPECT(group_waits_fit(true, &word, 240, 256));
  EXPECT(group_waits_fit(true, &word, 256, 256));
  EXPECT(!group_waits_fit(true, &word, 257, 256));
  EXPECT(!group_waits_fit(false, &word, 240, 256));
  EXPECT(!group_waits_fit(true, nullptr, 240, 256));
  EXPECT(!group_waits_fit(true, &word, 0, 256));
  if (fails == 0) std::printf("ok\n");
  return fails == 0 ? 0 : 1;
}
