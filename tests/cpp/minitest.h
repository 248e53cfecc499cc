// minitest.h - a small gtest-compatible subset (TEST, TEST_F, EXPECT_* /
// ASSERT_*, streamed messages, ASSERT_NO_FATAL_FAILURE) so the restated
// specification suites read like the reference's GoogleTest files without a
// network fetch. Each binary's main() is RUN_ALL_TESTS(argc, argv): optional
// arguments are suite-name filters; the exit code is the number of failed tests.
#pragma once

#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <iostream>
#include <optional>
#include <sstream>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

namespace minitest {

struct TestInfo {
    std::string suite;
    std::string name;
    std::function<void()> run;
};

inline std::vector<TestInfo>& registry() {
    static std::vector<TestInfo> tests;
    return tests;
}

struct State {
    int failures = 0;  // checks failed in the current test
    int fatal = 0;     // fatal checks failed in the current test
};

inline State& state() {
    static State s;
    return s;
}

struct Registrar {
    Registrar(const char* suite, const char* name, std::function<void()> fn) {
        registry().push_back({suite, name, std::move(fn)});
    }
};

class Test {
public:
    virtual ~Test() = default;
    virtual void SetUp() {}
    virtual void TearDown() {}
    virtual void TestBody() = 0;
};

template <typename T, typename = void>
struct Printable : std::false_type {};
template <typename T>
struct Printable<T, std::void_t<decltype(std::declval<std::ostream&>() << std::declval<const T&>())>>
    : std::true_type {};

template <typename T>
struct IsOptional : std::false_type {};
template <typename T>
struct IsOptional<std::optional<T>> : std::true_type {};
template <typename T>
struct IsVector : std::false_type {};
template <typename T, typename A>
struct IsVector<std::vector<T, A>> : std::true_type {};

template <typename T>
std::string show(const T& v) {
    if constexpr (IsOptional<T>::value) {
        return v.has_value() ? show(*v) : std::string("nullopt");
    } else if constexpr (IsVector<T>::value) {
        std::string s = "{";
        for (std::size_t i = 0; i < v.size(); ++i) s += (i ? ", " : "") + show(v[i]);
        return s + "}";
    } else if constexpr (std::is_enum_v<T>) {
        return std::to_string(static_cast<long long>(v));
    } else if constexpr (std::is_same_v<T, std::byte>) {
        return std::to_string(static_cast<int>(v));
    } else if constexpr (Printable<T>::value) {
        std::ostringstream os;
        os << v;
        return os.str();
    } else {
        return "<unprintable>";
    }
}

class Message {
public:
    template <typename T>
    Message& operator<<(const T& v) {
        os_ << show(v);
        return *this;
    }
    Message& operator<<(const char* s) {
        os_ << s;
        return *this;
    }
    std::string str() const { return os_.str(); }

private:
    std::ostringstream os_;
};

// Records a failed check; used as `helper = Message() << ...` so a streamed
// message can follow the macro, and `return helper = ...` for fatal checks.
class Failure {
public:
    Failure(const char* file, int line, std::string what, bool fatal)
        : file_(file), line_(line), what_(std::move(what)), fatal_(fatal) {}
    void operator=(const Message& m) const {
        state().failures += 1;
        if (fatal_) state().fatal += 1;
        std::cout << file_ << ":" << line_ << ": Failure\n  " << what_;
        const std::string extra = m.str();
        if (!extra.empty()) std::cout << "\n  " << extra;
        std::cout << std::endl;
    }

private:
    const char* file_;
    int line_;
    std::string what_;
    bool fatal_;
};

template <typename A, typename B, typename Op>
bool compare(const A& a, const B& b, Op op, std::string& what, const char* ea, const char* eb, const char* sym) {
    if (op(a, b)) return true;
    what = std::string("Expected: ") + ea + " " + sym + " " + eb + "\n  Actual: " + show(a) + " vs " + show(b);
    return false;
}

inline bool near(double a, double b, double tol, std::string& what, const char* ea, const char* eb) {
    if (std::fabs(a - b) <= tol) return true;
    what = std::string("Expected |") + ea + " - " + eb + "| <= " + std::to_string(tol) + "\n  Actual: " +
           std::to_string(a) + " vs " + std::to_string(b);
    return false;
}

inline bool float_eq(float a, float b, std::string& what, const char* ea, const char* eb) {
    // Within 4 units in the last place, like gtest's EXPECT_FLOAT_EQ.
    if (a == b) return true;
    int32_t ia, ib;
    std::memcpy(&ia, &a, 4);
    std::memcpy(&ib, &b, 4);
    if (ia < 0) ia = static_cast<int32_t>(0x80000000u) - ia;
    if (ib < 0) ib = static_cast<int32_t>(0x80000000u) - ib;
    const long long d = static_cast<long long>(ia) - ib;
    if (!std::isnan(a) && !std::isnan(b) && (d < 0 ? -d : d) <= 4) return true;
    what = std::string("Expected float equality of ") + ea + " and " + eb + "\n  Actual: " + std::to_string(a) +
           " vs " + std::to_string(b);
    return false;
}

inline int run_all(int argc, char** argv) {
    int failed = 0, ran = 0;
    std::vector<std::string> failed_names;
    for (const TestInfo& t : registry()) {
        bool selected = argc <= 1;
        for (int i = 1; i < argc && !selected; ++i) selected = t.suite == argv[i];
        if (!selected) continue;
        ++ran;
        state() = State{};
        std::cout << "[ RUN      ] " << t.suite << "." << t.name << std::endl;
        t.run();
        if (state().failures == 0) {
            std::cout << "[       OK ] " << t.suite << "." << t.name << std::endl;
        } else {
            ++failed;
            failed_names.push_back(t.suite + "." + t.name);
            std::cout << "[  FAILED  ] " << t.suite << "." << t.name << std::endl;
        }
    }
    std::cout << "[==========] " << ran << " tests ran, " << (ran - failed) << " passed, " << failed << " failed"
              << std::endl;
    for (const std::string& n : failed_names) std::cout << "[  FAILED  ] " << n << std::endl;
    return failed;
}

}  // namespace minitest

namespace testing = minitest;

#define MT_CAT_(a, b) a##b
#define MT_CAT(a, b) MT_CAT_(a, b)

#define TEST(suite, name)                                                                          \
    static void MT_CAT(mt_body_##suite##_, name)();                                                \
    static ::minitest::Registrar MT_CAT(mt_reg_##suite##_, name)(#suite, #name,                    \
                                                                 &MT_CAT(mt_body_##suite##_, name)); \
    static void MT_CAT(mt_body_##suite##_, name)()

#define TEST_F(fixture, name)                                                                      \
    class MT_CAT(fixture##_, name##_Test) : public fixture {                                       \
    public:                                                                                        \
        void TestBody() override;                                                                  \
    };                                                                                             \
    static ::minitest::Registrar MT_CAT(mt_reg_##fixture##_, name)(#fixture, #name, [] {           \
        MT_CAT(fixture##_, name##_Test) t;                                                         \
        ::minitest::Test& base = t; /* SetUp/TearDown may be protected in the fixture */           \
        base.SetUp();                                                                              \
        if (::minitest::state().fatal == 0) base.TestBody();                                       \
        base.TearDown();                                                                           \
    });                                                                                            \
    void MT_CAT(fixture##_, name##_Test)::TestBody()

#define MT_CHECK(ok, what, fatal) \
    if (ok) {                     \
    } else                        \
        fatal ::minitest::Failure(__FILE__, __LINE__, what, true) = ::minitest::Message()

#define MT_FATAL return
#define MT_NONFATAL

#define MT_BOOL(cond, expect, fatal_kw, fatal)                                                          \
    if (static_cast<bool>(cond) == (expect)) {                                                          \
    } else                                                                                              \
        fatal_kw ::minitest::Failure(__FILE__, __LINE__,                                                \
                                     std::string("Expected ") + #cond + " to be " + ((expect) ? "true" : "false"), \
                                     fatal) = ::minitest::Message()

#define EXPECT_TRUE(c) MT_BOOL(c, true, MT_NONFATAL, false)
#define EXPECT_FALSE(c) MT_BOOL(c, false, MT_NONFATAL, false)
#define ASSERT_TRUE(c) MT_BOOL(c, true, MT_FATAL, true)
#define ASSERT_FALSE(c) MT_BOOL(c, false, MT_FATAL, true)

#define MT_CMP(a, b, op, sym, fatal_kw, fatal)                                                           \
    if (std::string mt_what_;                                                                            \
        ::minitest::compare((a), (b), [](const auto& x, const auto& y) { return x op y; }, mt_what_, #a, \
                            #b, sym)) {                                                                  \
    } else                                                                                               \
        fatal_kw ::minitest::Failure(__FILE__, __LINE__, mt_what_, fatal) = ::minitest::Message()

#define EXPECT_EQ(a, b) MT_CMP(a, b, ==, "==", MT_NONFATAL, false)
#define EXPECT_NE(a, b) MT_CMP(a, b, !=, "!=", MT_NONFATAL, false)
#define EXPECT_LT(a, b) MT_CMP(a, b, <, "<", MT_NONFATAL, false)
#define EXPECT_LE(a, b) MT_CMP(a, b, <=, "<=", MT_NONFATAL, false)
#define EXPECT_GT(a, b) MT_CMP(a, b, >, ">", MT_NONFATAL, false)
#define EXPECT_GE(a, b) MT_CMP(a, b, >=, ">=", MT_NONFATAL, false)
#define ASSERT_EQ(a, b) MT_CMP(a, b, ==, "==", MT_FATAL, true)
#define ASSERT_NE(a, b) MT_CMP(a, b, !=, "!=", MT_FATAL, true)
#define ASSERT_LT(a, b) MT_CMP(a, b, <, "<", MT_FATAL, true)
#define ASSERT_LE(a, b) MT_CMP(a, b, <=, "<=", MT_FATAL, true)
#define ASSERT_GT(a, b) MT_CMP(a, b, >, ">", MT_FATAL, true)
#define ASSERT_GE(a, b) MT_CMP(a, b, >=, ">=", MT_FATAL, true)

#define EXPECT_NEAR(a, b, tol)                                                                           \
    if (std::string mt_what_; ::minitest::near((a), (b), (tol), mt_what_, #a, #b)) {                     \
    } else                                                                                               \
        ::minitest::Failure(__FILE__, __LINE__, mt_what_, false) = ::minitest::Message()
#define ASSERT_NEAR(a, b, tol)                                                                           \
    if (std::string mt_what_; ::minitest::near((a), (b), (tol), mt_what_, #a, #b)) {                     \
    } else                                                                                               \
        return ::minitest::Failure(__FILE__, __LINE__, mt_what_, true) = ::minitest::Message()
#define EXPECT_FLOAT_EQ(a, b)                                                                            \
    if (std::string mt_what_; ::minitest::float_eq((a), (b), mt_what_, #a, #b)) {                        \
    } else                                                                                               \
        ::minitest::Failure(__FILE__, __LINE__, mt_what_, false) = ::minitest::Message()

#define ASSERT_NO_FATAL_FAILURE(stmt)                        \
    do {                                                     \
        const int mt_before_ = ::minitest::state().fatal;    \
        stmt;                                                \
        if (::minitest::state().fatal != mt_before_) return; \
    } while (0)

#define RUN_ALL_TESTS(argc, argv) ::minitest::run_all(argc, argv)
