// `oxmera doctor`: what this machine can and cannot do, with ROCm detection.
//
// Same command line, report shape, rendering and determinism contract as the
// reference CLI (crates/oxmera-cli/src/main.rs:1-39, doctor.rs:1-136,
// report.rs:1-50, probe.rs:1-72): `oxmera doctor [--fixture <path>]`,
// `oxmera --version`; a fixture (TOML) always renders the same bytes.
//
// What it adds: ROCm.  The reference detects CUDA only (nvidia-smi / nvcc on
// PATH, probe.rs:53-58).  Here the probe also records `hipcc --version` and
// the gfx targets `rocminfo` lists, and the report renders an AMD tier-2 line,
// a hipcc tool line and a `rocm` backend path naming whether a gfx950 device
// (the one this backend is built for) is visible.  Those lines appear when
// the report has a `gpu.rocm` key -- always when probed, and in fixtures
// that set it -- so a fixture without it renders exactly as the reference
// does.
//
// Fixtures are parsed by a small TOML reader that covers what the reports
// use: comments, [table], [[array-of-tables]], and string / boolean / integer
// / string-array values.

#include <fcntl.h>
#include <sys/stat.h>
#include <sys/utsname.h>
#include <sys/wait.h>
#include <unistd.h>

#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <map>
#include <optional>
#include <sstream>
#include <string>
#include <vector>

namespace {

constexpr const char *kVersion = "0.0.3";
constexpr const char *kUsage = "usage: oxmera <doctor [--fixture <path>] | --version>";

// ---- the report (report.rs:7-50, plus the ROCm fields) ----------------------------

struct Rung {
    std::string id, name, status;
};

struct Report {
    std::string os, arch;
    std::optional<std::string> rustc, cargo, just, reconverge, launchbound, hipcc;
    bool container = false;
    bool metal = false, cuda = false;
    std::optional<bool> rocm;         // present: render the ROCm lines
    std::vector<std::string> gfx;     // gfx targets rocminfo lists
    std::vector<Rung> ladder;
    bool ladder_found = false;
};

// ---- a small TOML reader -----------------------------------------------------------

struct Value {
    enum Kind { Str, Bool, Int, StrArray } kind = Str;
    std::string s;
    bool b = false;
    long long i = 0;
    std::vector<std::string> arr;
};

using Table = std::map<std::string, Value>;

struct Doc {
    Table root;
    std::map<std::string, Table> tables;
    std::map<std::string, std::vector<Table>> arrays;
};

struct ParseError {
    std::string msg;
};

void skip_ws(const std::string &l, size_t &p) {
    while (p < l.size() && (l[p] == ' ' || l[p] == '\t')) ++p;
}

void append_utf8(std::string &out, unsigned cp) {
    if (cp < 0x80) {
        out += (char)cp;
    } else if (cp < 0x800) {
        out += (char)(0xC0 | (cp >> 6));
        out += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
        out += (char)(0xE0 | (cp >> 12));
        out += (char)(0x80 | ((cp >> 6) & 0x3F));
        out += (char)(0x80 | (cp & 0x3F));
    } else {
        out += (char)(0xF0 | (cp >> 18));
        out += (char)(0x80 | ((cp >> 12) & 0x3F));
        out += (char)(0x80 | ((cp >> 6) & 0x3F));
        out += (char)(0x80 | (cp & 0x3F));
    }
}

std::string parse_string(const std::string &l, size_t &p, int line) {
    const char q = l[p++];
    std::string out;
    while (p < l.size() && l[p] != q) {
        char c = l[p++];
        if (q == '"' && c == '\\') {
            if (p >= l.size()) break;
            const char e = l[p++];
            switch (e) {
            case 'n': out += '\n'; break;
            case 't': out += '\t'; break;
            case 'r': out += '\r'; break;
            case '"': out += '"'; break;
            case '\\': out += '\\'; break;
            case 'u':
            case 'U': {
                const size_t n = e == 'u' ? 4 : 8;
                if (p + n > l.size()) throw ParseError{"line " + std::to_string(line) + ": bad escape"};
                append_utf8(out, (unsigned)std::stoul(l.substr(p, n), nullptr, 16));
                p += n;
                break;
            }
            default: throw ParseError{"line " + std::to_string(line) + ": unknown escape \\" + std::string(1, e)};
            }
        } else {
            out += c;
        }
    }
    if (p >= l.size()) throw ParseError{"line " + std::to_string(line) + ": unterminated string"};
    ++p;
    return out;
}

Value parse_value(const std::string &l, size_t &p, int line) {
    Value v;
    skip_ws(l, p);
    if (p >= l.size()) throw ParseError{"line " + std::to_string(line) + ": missing value"};
    if (l[p] == '"' || l[p] == '\'') {
        v.kind = Value::Str;
        v.s = parse_string(l, p, line);
    } else if (l.compare(p, 4, "true") == 0) {
        v.kind = Value::Bool;
        v.b = true;
        p += 4;
    } else if (l.compare(p, 5, "false") == 0) {
        v.kind = Value::Bool;
        v.b = false;
        p += 5;
    } else if (l[p] == '[') {
        v.kind = Value::StrArray;
        ++p;
        for (;;) {
            skip_ws(l, p);
            if (p < l.size() && l[p] == ']') {
                ++p;
                break;
            }
            if (p >= l.size() || (l[p] != '"' && l[p] != '\''))
                throw ParseError{"line " + std::to_string(line) + ": only arrays of strings are supported"};
            v.arr.push_back(parse_string(l, p, line));
            skip_ws(l, p);
            if (p < l.size() && l[p] == ',') ++p;
        }
    } else {
        size_t q = p;
        if (q < l.size() && (l[q] == '-' || l[q] == '+')) ++q;
        size_t d = q;
        while (d < l.size() && (isdigit((unsigned char)l[d]) || l[d] == '_')) ++d;
        if (d == q) throw ParseError{"line " + std::to_string(line) + ": unsupported value"};
        std::string digits;
        for (size_t k = p; k < d; ++k)
            if (l[k] != '_') digits += l[k];
        v.kind = Value::Int;
        v.i = std::stoll(digits);
        p = d;
    }
    return v;
}

Doc parse_toml(const std::string &text) {
    Doc doc;
    Table *cur = &doc.root;
    std::istringstream in(text);
    std::string l;
    int line = 0;
    while (std::getline(in, l)) {
        ++line;
        size_t p = 0;
        skip_ws(l, p);
        if (p >= l.size() || l[p] == '#') continue;
        if (l[p] == '[') {
            const bool arr = l.compare(p, 2, "[[") == 0;
            const size_t open = p + (arr ? 2 : 1);
            const size_t close = l.find(arr ? "]]" : "]", open);
            if (close == std::string::npos) throw ParseError{"line " + std::to_string(line) + ": unclosed table header"};
            std::string name = l.substr(open, close - open);
            while (!name.empty() && name.back() == ' ') name.pop_back();
            while (!name.empty() && name.front() == ' ') name.erase(name.begin());
            if (arr) {
                doc.arrays[name].emplace_back();
                cur = &doc.arrays[name].back();
            } else {
                if (doc.tables.count(name)) throw ParseError{"line " + std::to_string(line) + ": duplicate table [" + name + "]"};
                cur = &doc.tables[name];
            }
            continue;
        }
        const size_t eq = l.find('=', p);
        if (eq == std::string::npos) throw ParseError{"line " + std::to_string(line) + ": expected key = value"};
        std::string key = l.substr(p, eq - p);
        while (!key.empty() && (key.back() == ' ' || key.back() == '\t')) key.pop_back();
        if (key.size() >= 2 && key.front() == '"' && key.back() == '"') key = key.substr(1, key.size() - 2);
        size_t q = eq + 1;
        Value v = parse_value(l, q, line);
        skip_ws(l, q);
        if (q < l.size() && l[q] != '#') throw ParseError{"line " + std::to_string(line) + ": trailing characters"};
        if (cur->count(key)) throw ParseError{"line " + std::to_string(line) + ": duplicate key `" + key + "`"};
        (*cur)[key] = v;
    }
    return doc;
}

// typed field access with serde-like messages
const Value *field(const Table &t, const std::string &k) {
    auto it = t.find(k);
    return it == t.end() ? nullptr : &it->second;
}

std::string req_str(const Table &t, const std::string &k) {
    const Value *v = field(t, k);
    if (!v) throw ParseError{"missing field `" + k + "`"};
    if (v->kind != Value::Str) throw ParseError{"invalid type for `" + k + "`: expected a string"};
    return v->s;
}

std::optional<std::string> opt_str(const Table &t, const std::string &k) {
    const Value *v = field(t, k);
    if (!v) return std::nullopt;
    if (v->kind != Value::Str) throw ParseError{"invalid type for `" + k + "`: expected a string"};
    return v->s;
}

bool req_bool(const Table &t, const std::string &k) {
    const Value *v = field(t, k);
    if (!v) throw ParseError{"missing field `" + k + "`"};
    if (v->kind != Value::Bool) throw ParseError{"invalid type for `" + k + "`: expected a boolean"};
    return v->b;
}

std::optional<bool> opt_bool(const Table &t, const std::string &k) {
    const Value *v = field(t, k);
    if (!v) return std::nullopt;
    if (v->kind != Value::Bool) throw ParseError{"invalid type for `" + k + "`: expected a boolean"};
    return v->b;
}

Report report_from(const Doc &d) {
    Report r;
    r.os = req_str(d.root, "os");
    r.arch = req_str(d.root, "arch");
    if (auto lf = opt_bool(d.root, "ladder_found")) r.ladder_found = *lf;
    auto tc = d.tables.find("toolchain");
    if (tc == d.tables.end()) throw ParseError{"missing field `toolchain`"};
    r.rustc = opt_str(tc->second, "rustc");
    r.cargo = opt_str(tc->second, "cargo");
    r.just = opt_str(tc->second, "just");
    r.reconverge = opt_str(tc->second, "reconverge");
    r.launchbound = opt_str(tc->second, "launchbound");
    r.hipcc = opt_str(tc->second, "hipcc");
    r.container = req_bool(tc->second, "container");
    auto gpu = d.tables.find("gpu");
    if (gpu == d.tables.end()) throw ParseError{"missing field `gpu`"};
    r.metal = req_bool(gpu->second, "metal");
    r.cuda = req_bool(gpu->second, "cuda");
    r.rocm = opt_bool(gpu->second, "rocm");
    if (const Value *g = field(gpu->second, "gfx")) {
        if (g->kind != Value::StrArray) throw ParseError{"invalid type for `gfx`: expected an array of strings"};
        r.gfx = g->arr;
    }
    auto lad = d.arrays.find("ladder");
    if (lad != d.arrays.end())
        for (const Table &t : lad->second) r.ladder.push_back({req_str(t, "id"), req_str(t, "name"), req_str(t, "status")});
    return r;
}

// ---- probing the real machine (probe.rs:11-72) --------------------------------------

bool on_path(const std::string &cmd) {
    const char *path = std::getenv("PATH");
    if (!path) return false;
    std::string p(path);
    size_t s = 0;
    for (;;) {
        const size_t e = p.find(':', s);
        std::string dir = p.substr(s, e == std::string::npos ? std::string::npos : e - s);
        if (dir.empty()) dir = ".";
        const std::string f = dir + "/" + cmd;
        struct stat st {};
        if (stat(f.c_str(), &st) == 0 && S_ISREG(st.st_mode)) return true;
        if (e == std::string::npos) return false;
        s = e + 1;
    }
}

// stdout of `cmd args...` (no shell), or nullopt when it cannot run or fails
std::optional<std::string> run_capture(const std::string &cmd, const std::vector<std::string> &args) {
    int fd[2];
    if (pipe(fd) != 0) return std::nullopt;
    const pid_t pid = fork();
    if (pid < 0) {
        close(fd[0]);
        close(fd[1]);
        return std::nullopt;
    }
    if (pid == 0) {
        dup2(fd[1], 1);
        const int devnull = open("/dev/null", O_WRONLY);
        if (devnull >= 0) dup2(devnull, 2);
        close(fd[0]);
        close(fd[1]);
        std::vector<char *> argv{const_cast<char *>(cmd.c_str())};
        for (const auto &a : args) argv.push_back(const_cast<char *>(a.c_str()));
        argv.push_back(nullptr);
        execvp(cmd.c_str(), argv.data());
        _exit(127);
    }
    close(fd[1]);
    std::string out;
    char buf[4096];
    ssize_t n;
    while ((n = read(fd[0], buf, sizeof buf)) > 0) out.append(buf, (size_t)n);
    close(fd[0]);
    int status = 0;
    waitpid(pid, &status, 0);
    if (!WIFEXITED(status) || WEXITSTATUS(status) != 0) return std::nullopt;
    return out;
}

std::string trim(const std::string &s) {
    size_t a = 0, b = s.size();
    while (a < b && isspace((unsigned char)s[a])) ++a;
    while (b > a && isspace((unsigned char)s[b - 1])) --b;
    return s.substr(a, b - a);
}

std::optional<std::string> first_line_of(const std::string &cmd, const std::vector<std::string> &args) {
    auto out = run_capture(cmd, args);
    if (!out) return std::nullopt;
    std::istringstream in(*out);
    std::string l;
    if (!std::getline(in, l)) return std::nullopt;
    return trim(l);
}

// gfx targets rocminfo lists ("Name: gfx950"), first-seen order, unique
std::vector<std::string> rocminfo_gfx() {
    std::vector<std::string> gfx;
    auto out = run_capture("rocminfo", {});
    if (!out) return gfx;
    std::istringstream in(*out);
    std::string l;
    while (std::getline(in, l)) {
        const std::string t = trim(l);
        if (t.compare(0, 5, "Name:") != 0) continue;
        const std::string v = trim(t.substr(5));
        if (v.compare(0, 3, "gfx") != 0) continue;
        bool seen = false;
        for (const auto &g : gfx) seen = seen || g == v;
        if (!seen) gfx.push_back(v);
    }
    return gfx;
}

// exercises/manifest.toml in the working directory or the nearest parent
// that has one (probe.rs:24-45)
void find_ladder(Report &r) {
    char cwd[4096];
    if (!getcwd(cwd, sizeof cwd)) return;
    std::string d(cwd);
    for (;;) {
        const std::string cand = (d == "/" ? "" : d) + "/exercises/manifest.toml";
        struct stat st {};
        if (stat(cand.c_str(), &st) == 0 && S_ISREG(st.st_mode)) {
            std::ifstream f(cand);
            std::stringstream ss;
            ss << f.rdbuf();
            try {
                Doc doc = parse_toml(ss.str());
                auto ex = doc.arrays.find("exercise");
                if (ex != doc.arrays.end())
                    for (const Table &t : ex->second)
                        r.ladder.push_back({req_str(t, "id"), req_str(t, "name"), req_str(t, "status")});
                r.ladder_found = true;
            } catch (const ParseError &) {
                r.ladder.clear();
                r.ladder_found = false;
            }
            return;
        }
        if (d == "/") return;
        const size_t slash = d.find_last_of('/');
        d = slash == 0 ? "/" : d.substr(0, slash);
    }
}

Report probe() {
    Report r;
    struct utsname u {};
    uname(&u);
    r.os = u.sysname;
    for (auto &c : r.os) c = (char)tolower((unsigned char)c);
    if (r.os == "darwin") r.os = "macos";
    r.arch = u.machine;
    if (r.arch == "arm64") r.arch = "aarch64";
    r.metal = r.os == "macos" && r.arch == "aarch64";
    r.cuda = on_path("nvidia-smi") || on_path("nvcc");
    r.rustc = first_line_of("rustc", {"--version"});
    r.cargo = first_line_of("cargo", {"--version"});
    r.just = first_line_of("just", {"--version"});
    r.reconverge = first_line_of("cargo-reconverge", {"--version"});
    r.launchbound = first_line_of("launchbound", {"--version"});
    r.container = on_path("container") || on_path("docker");
    r.hipcc = first_line_of("hipcc", {"--version"});
    r.rocm = on_path("hipcc") || on_path("rocminfo");
    if (on_path("rocminfo")) r.gfx = rocminfo_gfx();
    find_ladder(r);
    return r;
}

// ---- rendering (doctor.rs:23-136) ---------------------------------------------------

// left-justify to `width` characters (UTF-8 aware, as Rust's {:<w})
std::string pad(const std::string &s, size_t width) {
    size_t chars = 0;
    for (unsigned char c : s) chars += (c & 0xC0) != 0x80;
    return chars >= width ? s : s + std::string(width - chars, ' ');
}

std::string tool_line(const std::string &name, const std::optional<std::string> &v) {
    return "  " + pad(name, 12) + " " + (v ? *v : std::string("not found"));
}

const char *status_mark(const std::string &s) {
    if (s == "solved") return "x";
    if (s == "todo") return " ";
    return ".";
}

std::string render(const Report &r) {
    std::string out;
    auto line = [&](const std::string &s) {
        out += s;
        out += '\n';
    };
    const bool amd = r.rocm.has_value();
    line("oxmera doctor");
    line("=============");
    line("");
    line("host: " + r.os + " / " + r.arch);
    line("");
    line("toolchain");
    line(tool_line("rustc", r.rustc));
    line(tool_line("cargo", r.cargo));
    line(tool_line("just", r.just));
    line(tool_line("reconverge", r.reconverge));
    line(tool_line("launchbound", r.launchbound));
    if (amd) line(tool_line("hipcc", r.hipcc));
    line("  " + pad("container", 12) + " " + (r.container ? "yes" : "no"));
    line("");

    const bool tier0 = r.rustc && r.cargo;
    const bool gate = tier0 && r.reconverge;
    line("tiers");
    line(std::string("  tier 0  edit / check / CPU backend        ") + (tier0 ? "available" : "MISSING rustc/cargo"));
    line(std::string("  tier 0  convergence gate (reconverge)     ") +
         (gate ? "available" : "install cargo-reconverge + reconverge-driver"));
    line(std::string("  tier 1  container PTX (cargo oxide)       ") +
         (r.container ? "available" : "no container runtime found"));
    line("  tier 2  NVIDIA execution                  metered \xe2\x80\x94 approved GPU sessions only");
    if (amd) line("  tier 2  AMD execution (hip-gfx950)        metered \xe2\x80\x94 approved GPU sessions only");
    line("");

    line("backend paths");
    line("  cpu     always available \xe2\x80\x94 the correctness ground truth");
    line(std::string("  metal   ") + (r.metal ? "plausible on this host" : "not on this host") +
         "  (no convergence gate exists on this path)");
    line(std::string("  cuda    ") + (r.cuda ? "toolkit visible" : "no toolkit here \xe2\x80\x94 tier 1/2 territory") +
         "  (verdicts and timings are per-part)");
    if (amd) {
        bool has950 = false;
        std::string list;
        for (const auto &g : r.gfx) {
            has950 = has950 || g == "gfx950";
            list += (list.empty() ? "" : ", ") + g;
        }
        std::string s;
        if (!*r.rocm)
            s = "no ROCm toolkit here";
        else if (has950)
            s = "gfx950 visible \xe2\x80\x94 the hip-gfx950 backend can run";
        else if (!r.gfx.empty())
            s = "toolkit visible, devices " + list + " \xe2\x80\x94 the hip-gfx950 backend needs gfx950";
        else
            s = "toolkit visible, no device listed \xe2\x80\x94 the hip-gfx950 backend cross-compiles only";
        line("  rocm    " + s + "  (one process per GPU)");
    }
    line("");

    line("exercise ladder");
    if (!r.ladder_found) {
        line("  no exercises/manifest.toml found from here");
    } else {
        int solved = 0, todo = 0, planned = 0;
        for (const auto &x : r.ladder) {
            solved += x.status == "solved";
            todo += x.status == "todo";
            planned += x.status == "planned";
        }
        line("  " + std::to_string(solved) + " solved, " + std::to_string(todo) + " todo, " + std::to_string(planned) +
             " planned");
        for (const auto &x : r.ladder) line(std::string("  [") + status_mark(x.status) + "] " + pad(x.id, 4) + " " + x.name);
    }
    line("");
    line("doctor: report complete");
    return out;
}

int doctor(const std::vector<std::string> &args) {
    Report r;
    if (args.empty()) {
        r = probe();
    } else if (args.size() == 2 && args[0] == "--fixture") {
        std::ifstream f(args[1]);
        if (!f.good()) {
            std::fprintf(stderr, "oxmera doctor: cannot read fixture %s: No such file or directory\n", args[1].c_str());
            return 1;
        }
        std::stringstream ss;
        ss << f.rdbuf();
        try {
            r = report_from(parse_toml(ss.str()));
        } catch (const ParseError &e) {
            std::fprintf(stderr, "oxmera doctor: cannot parse fixture %s: %s\n", args[1].c_str(), e.msg.c_str());
            return 1;
        }
    } else {
        std::fprintf(stderr, "oxmera doctor: usage: oxmera doctor [--fixture <path>]\n");
        return 1;
    }
    const std::string s = render(r);
    std::fwrite(s.data(), 1, s.size(), stdout);
    return 0;
}

}  // namespace

int main(int argc, char **argv) {
    std::vector<std::string> args(argv + 1, argv + argc);
    if (!args.empty() && (args[0] == "--version" || args[0] == "-V")) {
        std::printf("oxmera %s\n", kVersion);
        return 0;
    }
    if (!args.empty() && args[0] == "doctor") return doctor(std::vector<std::string>(args.begin() + 1, args.end()));
    std::fprintf(stderr, "%s\n", kUsage);
    return 1;
}
