// Locates tests/golden/ for the specification binaries: $QVP_GOLDEN_DIR when
// set, else relative to the executable (<root>/build/tests/<binary>).
#pragma once

#include <cstdlib>
#include <fstream>
#include <sstream>
#include <string>

#include <limits.h>
#include <unistd.h>
#include <zlib.h>

namespace golden {

inline std::string dir() {
    if (const char* env = std::getenv("QVP_GOLDEN_DIR")) return env;
    char buf[PATH_MAX];
    const ssize_t n = readlink("/proc/self/exe", buf, sizeof buf - 1);
    if (n <= 0) return "tests/golden";
    std::string exe(buf, static_cast<std::size_t>(n));
    for (int up = 0; up < 3; ++up) exe = exe.substr(0, exe.find_last_of('/'));
    return exe + "/tests/golden";
}

inline bool read(const std::string& name, std::string& out) {
    std::ifstream f(dir() + "/" + name);
    if (!f) return false;
    std::ostringstream ss;
    ss << f.rdbuf();
    out = ss.str();
    return true;
}

// A gzip-compressed fixture, decompressed.
inline bool read_gz(const std::string& name, std::string& out) {
    gzFile f = gzopen((dir() + "/" + name).c_str(), "rb");
    if (f == nullptr) return false;
    out.clear();
    char buf[1 << 16];
    int n = 0;
    while ((n = gzread(f, buf, sizeof buf)) > 0) out.append(buf, static_cast<std::size_t>(n));
    const bool ok = n == 0;
    gzclose(f);
    return ok;
}

// First differing line of two logs, for the failure message.
inline std::string first_difference(const std::string& a, const std::string& b) {
    std::istringstream x(a), y(b);
    std::string la, lb;
    for (int line = 1;; ++line) {
        const bool ga = static_cast<bool>(std::getline(x, la));
        const bool gb = static_cast<bool>(std::getline(y, lb));
        if (!ga && !gb) return "identical";
        if (la != lb || ga != gb) {
            return "line " + std::to_string(line) + ":\n    expected: " + (gb ? lb : "<end>") + "\n    actual:   " +
                   (ga ? la : "<end>");
        }
    }
}

}  // namespace golden
