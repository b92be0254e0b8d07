// Minimal checking helpers for the C++ API test programs.
#pragma once

#include <cstdio>
#include <exception>
#include <string>

namespace apitest {

inline int& failures() {
  static int n = 0;
  return n;
}

#define CHECK(cond)                                                              \
  do {                                                                           \
    if (!(cond)) {                                                               \
      std::fprintf(stderr, "%s:%d: CHECK failed: %s\n", __FILE__, __LINE__, #cond); \
      ++::apitest::failures();                                                   \
    }                                                                            \
  } while (0)

// Runs fn and checks that it throws E whose message contains `needle`.
template <typename E, typename Fn>
void expect_throw(const char* what, const std::string& needle, Fn&& fn) {
  try {
    fn();
  } catch (const E& e) {
    if (std::string(e.what()).find(needle) == std::string::npos) {
      std::fprintf(stderr, "%s: message '%s' lacks '%s'\n", what, e.what(), needle.c_str());
      ++failures();
    }
    return;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "%s: wrong exception type: %s\n", what, e.what());
    ++failures();
    return;
  }
  std::fprintf(stderr, "%s: no exception\n", what);
  ++failures();
}

inline int finish(const char* name) {
  if (failures()) {
    std::fprintf(stderr, "%s: %d failure(s)\n", name, failures());
    return 1;
  }
  std::printf("%s: all checks passed\n", name);
  return 0;
}

}  // namespace apitest
