// check.hpp -- minimal test harness for the C++ test programs: each TEST
// registers a function; main() runs them all (or those named on the command
// line) and exits non-zero if any CHECK failed.
#pragma once

#include <cmath>
#include <cstdio>
#include <functional>
#include <string>
#include <vector>

namespace check {

struct Case {
  const char *name;
  std::function<void()> fn;
};
inline std::vector<Case> &cases() {
  static std::vector<Case> c;
  return c;
}
inline int &failures() {
  static int f = 0;
  return f;
}
struct Register {
  Register(const char *name, std::function<void()> fn) { cases().push_back({name, std::move(fn)}); }
};

inline void fail(const char *file, int line, const std::string &what) {
  std::fprintf(stderr, "  FAILED %s:%d: %s\n", file, line, what.c_str());
  ++failures();
}

inline int run_all(int argc, char **argv) {
  int failed_cases = 0;
  for (const Case &c : cases()) {
    if (argc > 1) {
      bool wanted = false;
      for (int i = 1; i < argc; ++i) wanted |= std::string(argv[i]) == c.name;
      if (!wanted) continue;
    }
    const int before = failures();
    try {
      c.fn();
    } catch (const std::exception &e) {
      fail(__FILE__, __LINE__, std::string("unexpected exception: ") + e.what());
    }
    const bool ok = failures() == before;
    failed_cases += !ok;
    std::printf("%s %s\n", ok ? "PASS" : "FAIL", c.name);
    std::fflush(stdout);
  }
  std::printf("%d failed\n", failed_cases);
  return failed_cases ? 1 : 0;
}

}  // namespace check

#define TEST(name)                                               \
  static void name();                                            \
  static check::Register name##_reg(#name, name);               \
  static void name()

#define CHECK(cond)                                                    \
  do {                                                                 \
    if (!(cond)) check::fail(__FILE__, __LINE__, "CHECK(" #cond ")"); \
  } while (0)

#define CHECK_NEAR(a, b, tol)                                                              \
  do {                                                                                     \
    const double _a = (a), _b = (b);                                                       \
    if (!(std::fabs(_a - _b) <= (tol)))                                                    \
      check::fail(__FILE__, __LINE__,                                                      \
                  std::string(#a " = ") + std::to_string(_a) + " vs " + std::to_string(_b)); \
  } while (0)

// Expect `expr` to throw ammon::Error whose message contains `needle`.
#define CHECK_THROWS_WITH(expr, needle)                                                  \
  do {                                                                                   \
    bool _thrown = false;                                                                \
    try {                                                                                \
      expr;                                                                              \
    } catch (const ammon::Error &_e) {                                                   \
      _thrown = true;                                                                    \
      if (std::string(_e.what()).find(needle) == std::string::npos)                     \
        check::fail(__FILE__, __LINE__, std::string("message `") + _e.what() +          \
                                            "` lacks `" + (needle) + "`");               \
    }                                                                                    \
    if (!_thrown) check::fail(__FILE__, __LINE__, "expected an error from " #expr);     \
  } while (0)
