#pragma once
// Minimal test harness for the C++ front-end tests: TEST_CASE registers a
// function, CHECK records failures, CHECK_THROWS_WITH checks an exception's
// message.  `--list` prints the names; `--host-only` runs only the cases
// tagged HOST (no GPU launches); a name filter runs matching cases only.
#include <cstdio>
#include <cstring>
#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

namespace harness {

struct test {
  const char *name;
  bool host_only;
  std::function<void()> fn;
};

inline std::vector<test> &registry() {
  static std::vector<test> r;
  return r;
}
inline int &failures() {
  static int f = 0;
  return f;
}
inline const char *&current() {
  static const char *c = "";
  return c;
}

struct registrar {
  registrar(const char *n, bool host, std::function<void()> f) {
    registry().push_back({n, host, std::move(f)});
  }
};

inline void fail(const char *file, int line, const char *expr) {
  std::fprintf(stderr, "FAIL [%s] %s:%d: %s\n", current(), file, line, expr);
  failures()++;
}

inline int run(int argc, char **argv) {
  bool host_only = false, list = false;
  const char *filter = nullptr;
  for (int i = 1; i < argc; i++) {
    if (!std::strcmp(argv[i], "--host-only")) host_only = true;
    else if (!std::strcmp(argv[i], "--list")) list = true;
    else filter = argv[i];
  }
  int ran = 0;
  for (auto &t : registry()) {
    if (host_only && !t.host_only) continue;
    if (filter && !std::strstr(t.name, filter)) continue;
    if (list) {
      std::printf("%s\n", t.name);
      continue;
    }
    current() = t.name;
    std::printf("[case] %s\n", t.name);
    std::fflush(stdout);
    int before = failures();
    try {
      t.fn();
    } catch (std::exception &e) {
      std::fprintf(stderr, "FAIL [%s] unexpected exception: %s\n", t.name, e.what());
      failures()++;
    }
    std::printf("[%s] %s\n", failures() == before ? "ok" : "FAILED", t.name);
    ran++;
  }
  if (!list) std::printf("%d cases, %d failed checks\n", ran, failures());
  return failures() == 0 ? 0 : 1;
}

}  // namespace harness

#define HARNESS_CAT2(a, b) a##b
#define HARNESS_CAT(a, b) HARNESS_CAT2(a, b)
#define HARNESS_CASE(name, host)                                                          \
  static void HARNESS_CAT(case_, __LINE__)();                                             \
  static harness::registrar HARNESS_CAT(reg_, __LINE__)(name, host, HARNESS_CAT(case_, __LINE__)); \
  static void HARNESS_CAT(case_, __LINE__)()
#define TEST_CASE(name) HARNESS_CASE(name, false)
#define HOST_CASE(name) HARNESS_CASE(name, true)
#define CHECK(expr)                                   \
  do {                                                \
    if (!(expr)) harness::fail(__FILE__, __LINE__, #expr); \
  } while (0)
#define CHECK_THROWS_WITH(expr, msg)                                              \
  do {                                                                            \
    bool thrown_ = false;                                                         \
    try {                                                                         \
      (void)(expr);                                                               \
    } catch (std::exception & e_) {                                               \
      thrown_ = true;                                                             \
      if (std::string(e_.what()) != (msg)) harness::fail(__FILE__, __LINE__, #expr " message"); \
    }                                                                             \
    if (!thrown_) harness::fail(__FILE__, __LINE__, #expr " did not throw");      \
  } while (0)
