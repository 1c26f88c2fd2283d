// A minimal TEST / EXPECT harness in the style of the reference's gtest suites
// (kuiper/test/test_op/*.cpp): TEST(Suite, Name) registers a case, EXPECT_* records a
// failure and continues, ASSERT_* returns from the case.  Cases whose suite name
// starts with "Gpu" run only when the binary is started without --cpu-only.
#ifndef ORIN_MINI_TEST_H
#define ORIN_MINI_TEST_H

#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

namespace mini_test {

struct Case {
  const char* suite;
  const char* name;
  std::function<void()> fn;
};
inline std::vector<Case>& registry() {
  static std::vector<Case> r;
  return r;
}
inline int& failures() {
  static int f = 0;
  return f;
}
struct Registrar {
  Registrar(const char* s, const char* n, std::function<void()> f) {
    registry().push_back({s, n, std::move(f)});
  }
};

inline int run_all(int argc, char** argv) {
  bool cpu_only = false;
  const char* filter = nullptr;
  for (int i = 1; i < argc; ++i) {
    if (!strcmp(argv[i], "--cpu-only")) cpu_only = true;
    else filter = argv[i];
  }
  int run = 0, failed = 0;
  for (const Case& c : registry()) {
    if (cpu_only && !strncmp(c.suite, "Gpu", 3)) continue;
    const std::string full = std::string(c.suite) + "." + c.name;
    if (filter && full.find(filter) == std::string::npos) continue;
    printf("[ RUN      ] %s\n", full.c_str());
    fflush(stdout);
    const int before = failures();
    c.fn();
    const bool ok = failures() == before;
    printf("%s %s\n", ok ? "[       OK ]" : "[  FAILED  ]", full.c_str());
    fflush(stdout);
    ++run;
    failed += ok ? 0 : 1;
  }
  printf("[==========] %d tests ran, %d failed\n", run, failed);
  return failed ? 1 : 0;
}

}  // namespace mini_test

#define TEST(suite, name)                                                                  \
  static void suite##_##name##_body();                                                     \
  static mini_test::Registrar suite##_##name##_reg(#suite, #name, suite##_##name##_body);  \
  static void suite##_##name##_body()

#define EXPECT_TRUE(c)                                                                     \
  do {                                                                                     \
    if (!(c)) {                                                                            \
      printf("%s:%d: expected %s\n", __FILE__, __LINE__, #c);                              \
      ++mini_test::failures();                                                             \
    }                                                                                      \
  } while (0)
#define ASSERT_TRUE(c)                                                                     \
  do {                                                                                     \
    if (!(c)) {                                                                            \
      printf("%s:%d: required %s\n", __FILE__, __LINE__, #c);                              \
      ++mini_test::failures();                                                             \
      return;                                                                              \
    }                                                                                      \
  } while (0)
#define EXPECT_EQ(a, b) EXPECT_TRUE((a) == (b))
#define ASSERT_EQ(a, b) ASSERT_TRUE((a) == (b))

#endif  // ORIN_MINI_TEST_H
