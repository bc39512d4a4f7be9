// cli_common.h -- the pieces both command-line encoders share: a
// table-driven option parser (each option names its target; the usage text
// is generated from the same table), whole-file raw I/O on POSIX
// descriptors, and the stdout summary of an embedding.
//
// Exit-code convention of both tools: 0 ok (and --help), 1 a load, read,
// preprocess or encode failure, 2 bad arguments.
#pragma once

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace s2xcli {

enum { EXIT_OK = 0, EXIT_FAIL = 1, EXIT_USAGE = 2 };

// One command-line option.  Exactly one target is set: `text` (a string
// value), `number` (an int value), `grid` (two ints written "A,B"); none of
// them for a flag that only prints help.
struct Option {
    const char *name;   // "--model"
    const char *alias;  // "-m", or nullptr
    const char *meta;   // value placeholder for the usage text, nullptr for a flag
    const char *help;
    std::string *text = nullptr;
    int *number = nullptr;
    int *grid = nullptr;  // int[2]
};

enum class Parsed { ok, help, bad };

inline const Option *find_option(const std::vector<Option> &table, const char *arg) {
    for (const Option &o : table)
        if (!std::strcmp(arg, o.name) || (o.alias && !std::strcmp(arg, o.alias))) return &o;
    return nullptr;
}

// "A,B" with two integers; false if either is missing
inline bool read_grid(const char *s, int out[2]) {
    char *end = nullptr;
    errno = 0;
    const long a = std::strtol(s, &end, 10);
    if (end == s || *end != ',') return false;
    const char *second = end + 1;
    const long b = std::strtol(second, &end, 10);
    if (end == second || errno) return false;
    out[0] = (int)a;
    out[1] = (int)b;
    return true;
}

// Walks argv against the table.  `err` gets the message of a bad argument.
inline Parsed parse(int argc, char **argv, const std::vector<Option> &table, std::string &err) {
    int i = 1;
    while (i < argc) {
        const char *arg = argv[i++];
        if (!std::strcmp(arg, "--help") || !std::strcmp(arg, "-h")) return Parsed::help;
        const Option *o = find_option(table, arg);
        if (!o || (o->meta && i >= argc)) {
            err = std::string("Unknown arg: ") + arg;
            return Parsed::bad;
        }
        if (!o->meta) continue;
        const char *val = argv[i++];
        if (o->text) {
            *o->text = val;
        } else if (o->number) {
            *o->number = std::atoi(val);
        } else if (o->grid && !read_grid(val, o->grid)) {
            err = std::string(o->name) + " expects H,W (got: " + val + ")";
            return Parsed::bad;
        }
    }
    return Parsed::ok;
}

inline void print_usage(FILE *f, const char *title, const std::vector<std::string> &synopsis,
                        const std::vector<Option> &table) {
    std::fprintf(f, "%s\n\nUsage:\n", title);
    for (const std::string &line : synopsis) std::fprintf(f, "  %s\n", line.c_str());
    std::fprintf(f, "\nOptions:\n");
    for (const Option &o : table) {
        std::string left = o.name;
        if (o.alias) left += std::string(", ") + o.alias;
        if (o.meta) left += std::string(" ") + o.meta;
        std::fprintf(f, "  %-28s %s\n", left.c_str(), o.help);
    }
    std::fprintf(f, "  %-28s %s\n", "--help, -h", "this text");
}

// The whole file at `path` into `bytes`.
inline bool slurp(const std::string &path, std::vector<uint8_t> &bytes, std::string &err) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) {
        err = "could not open: " + path;
        return false;
    }
    struct stat st;
    bool ok = ::fstat(fd, &st) == 0;
    if (ok) {
        bytes.assign((size_t)st.st_size, 0);
        size_t done = 0;
        while (ok && done < bytes.size()) {
            const ssize_t n = ::read(fd, bytes.data() + done, bytes.size() - done);
            if (n < 0 && errno == EINTR) continue;
            ok = n > 0;
            done += ok ? (size_t)n : 0;
        }
    }
    ::close(fd);
    if (!ok) err = "could not read: " + path;
    return ok;
}

inline bool spill(const std::string &path, const void *data, size_t n_bytes, std::string &err) {
    const int fd = ::open(path.c_str(), O_WRONLY | O_CREAT | O_TRUNC, 0644);
    bool ok = fd >= 0;
    const uint8_t *p = static_cast<const uint8_t *>(data);
    size_t done = 0;
    while (ok && done < n_bytes) {
        const ssize_t n = ::write(fd, p + done, n_bytes - done);
        if (n < 0 && errno == EINTR) continue;
        ok = n > 0;
        done += ok ? (size_t)n : 0;
    }
    if (fd >= 0 && ::close(fd) != 0) ok = false;
    if (!ok) err = "could not write: " + path;
    return ok;
}

// A file of n_bytes reinterpreted as T values (n_bytes a multiple of sizeof T).
template <class T>
std::vector<T> as_values(const std::vector<uint8_t> &bytes) {
    std::vector<T> v(bytes.size() / sizeof(T));
    if (!v.empty()) std::memcpy(v.data(), bytes.data(), v.size() * sizeof(T));
    return v;
}

// One line for an embedding written to stdout: its size, L2 norm and the
// values at both ends.
inline void print_summary(FILE *f, const char *label, const std::vector<float> &e) {
    double ss = 0.0;
    for (float x : e) ss += (double)x * x;
    std::fprintf(f, "%s: dim %zu, L2 norm %.6g\n", label, e.size(), std::sqrt(ss));
    const size_t head = e.size() < 8 ? e.size() : 8;
    std::fprintf(f, "  first:");
    for (size_t i = 0; i < head; ++i) std::fprintf(f, " %.7g", e[i]);
    std::fprintf(f, "\n");
    if (e.size() > head) {
        std::fprintf(f, "  last: ");
        for (size_t i = e.size() - (e.size() - head < 4 ? e.size() - head : 4); i < e.size(); ++i)
            std::fprintf(f, " %.7g", e[i]);
        std::fprintf(f, "\n");
    }
}

}  // namespace s2xcli
