// test_numparse.cpp -- checks the CSV number conversions (numparse.hpp,
// compiled for the host) against the C library they restate: glibc's strtof
// and strtol, through libstdc++'s std::stof / std::stoi contract (nothing
// converted -> invalid; ERANGE, or an int out of range -> out of range).
//
// Usage: test_numparse [n_random] [seed].  Prints the first mismatches and
// exits non-zero if there is any.
#include <cerrno>
#include <cinttypes>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "numparse.hpp"
#include "numparse_table.hpp"

using namespace tg::numparse;

namespace {

Pow10Entry g_tab[kPow10Count];
long g_checked = 0, g_bad = 0;

uint32_t f2u(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}
float u2f(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

void check_float(const std::string& s) {
    const char* c = s.c_str();
    char* end = nullptr;
    errno = 0;
    const float f = std::strtof(c, &end);
    const int err = errno;
    // the field as the reference sees it: the C string up to the first NUL
    const size_t clen = std::strlen(c);
    int want = end == c ? kInvalid : (err == ERANGE ? kRange : kOk);
    uint32_t got_bits = 0xdeadbeef;
    const auto* p = reinterpret_cast<const unsigned char*>(s.data());
    const int got = parse_float(p, p + s.size(), g_tab, &got_bits);
    (void)clen;
    ++g_checked;
    bool ok = got == want && (want == kInvalid || got_bits == f2u(f));
    if (!ok) {
        if (g_bad < 40)
            std::printf("float mismatch: '%s' -> want status %d bits %08x, got status %d bits %08x\n",
                        s.c_str(), want, f2u(f), got, got_bits);
        ++g_bad;
    }
}

void check_int(const std::string& s) {
    const char* c = s.c_str();
    char* end = nullptr;
    errno = 0;
    const long v = std::strtol(c, &end, 10);
    const int err = errno;
    int want;
    if (end == c) want = kInvalid;
    else if (err == ERANGE || v < INT_MIN || v > INT_MAX) want = kRange;
    else want = kOk;
    int32_t got_v = 0x5a5a5a5a;
    const auto* p = reinterpret_cast<const unsigned char*>(s.data());
    const int got = parse_int(p, p + s.size(), &got_v);
    ++g_checked;
    if (got != want || (want == kOk && got_v != int32_t(v))) {
        if (g_bad < 40)
            std::printf("int mismatch: '%s' -> want status %d value %ld, got status %d value %d\n",
                        s.c_str(), want, v, got, got_v);
        ++g_bad;
    }
}

std::string fmt(const char* f, double v) {
    char buf[512];
    std::snprintf(buf, sizeof buf, f, v);
    return buf;
}
std::string fmti(const char* f, int prec, double v) {
    char buf[1024];
    std::snprintf(buf, sizeof buf, f, prec, v);
    return buf;
}

// All decimal forms around a float: shortest-ish, long, exact midpoints to
// either side and their truncations/perturbations.
void around(float x, std::mt19937_64& rng) {
    if (!std::isfinite(x)) return;
    const double d = x;
    for (int prec : {6, 8, 9, 12, 17, 25}) check_float(fmti("%.*g", prec, d));
    check_float(fmti("%.*e", 40, d));
    const float up = std::nextafterf(x, INFINITY), dn = std::nextafterf(x, -INFINITY);
    for (float nb : {up, dn}) {
        if (!std::isfinite(nb)) continue;
        const double mid = (d + double(nb)) / 2;  // exact in double
        const std::string exact = fmti("%.*e", 130, mid);
        check_float(exact);
        // truncations of the exact midpoint expansion and +-1 in the last kept digit
        const size_t epos = exact.find('e');
        const std::string mant = exact.substr(0, epos), ex = exact.substr(epos);
        for (int keep : {10, 12, 16, 19, 20, 22, 30, 50, 90}) {
            if (size_t(keep) + 2 >= mant.size()) continue;
            std::string t = mant.substr(0, size_t(keep) + 2);
            check_float(t + ex);
            std::string t2 = t;
            for (size_t i = t2.size(); i-- > 0;) {  // +1 ulp of the decimal
                if (t2[i] == '.' || t2[i] == '-') continue;
                if (t2[i] == '9') { t2[i] = '0'; continue; }
                ++t2[i];
                break;
            }
            check_float(t2 + ex);
            check_float(t + std::string(size_t(rng() % 5 + 1), '0') + "1" + ex);
        }
    }
}

std::string rand_digits(std::mt19937_64& rng, int n) {
    std::string s;
    for (int i = 0; i < n; ++i) s.push_back(char('0' + rng() % 10));
    return s;
}

}  // namespace

int main(int argc, char** argv) {
    const long n_random = argc > 1 ? std::atol(argv[1]) : 200000;
    const uint64_t seed = argc > 2 ? std::strtoull(argv[2], nullptr, 10) : 12345;
    build_pow10_table(g_tab);
    std::mt19937_64 rng(seed);

    // 1. hand-picked forms (syntax, specials, boundaries)
    const char* fixed[] = {
        "", " ", ".", "+", "-", "+.", "e5", ".e1", "1", "-1", "+1", "0", "-0", "00", "0.0",
        ".5", "5.", "1e", "1e+", "1e-", "1E5", "1e+05", "1e-05", "  \t\n\v\f\r 7", "1.5abc",
        "1..5", "1.5.5", "--1", "+-1", "0x", "0X", "0x.", "0x.8", "0xg", "0x1p", "0x1p+",
        "0x1P-3", "0X1.8p1", "0x.1", "0x1.fffffep127", "0x1.ffffffp127", "0x1p128",
        "0x1p-126", "0x1p-149", "0x1p-150", "0x1.8p-150", "0x1.fffffep-127", "0x1.ffffffp-127",
        "0x1.fffffefp-127", "0x1.fffffe8p-127", "0x1.fffffe00000000000000001p-127",
        "0x0.000000000000000000000000000001p0", "0x123456789abcdef0123p-70",
        "inf", "INF", "-inf", "infinity", "-Infinity", "infin", "in", "i", "infx",
        "nan", "NAN", "-nan", "nan(", "nan()", "nan(0)", "nan(123)", "nan(0x123)", "nan(0123)",
        "nan(08)", "nan(0x)", "nan(abc)", "nan(1_a)", "nan( 5)", "nan(+5)", "-nan(5)",
        "nan(0xffffffff)", "nan(4194303)", "nan(4194304)", "nan(99999999999999999999999)",
        "nan(0xfffffffffffffffffffff)", "nan(99999999999999999999999_)", "na", "n",
        "3.4028235e38", "3.4028236e38", "3.40282356e38", "3.40282357e38", "3.4028235677973366e38",
        "3.4028235677973365e38", "3.4028235677973367e38", "1e39", "1e38", "-1e39",
        "1.1754943508222875e-38", "1.17549435e-38", "1.1754943e-38", "1.17549433e-38",
        "1.1754943158e-38", "1.1754943157e-38", "1.17549431578982e-38", "1.17549431579e-38",
        "1.4e-45", "1.401298464324817e-45", "7e-46", "7.006e-46", "7.0064923216240854e-46",
        "7.0064923216240855e-46", "7.0064923216240853e-46", "1e-45", "1e-46", "1e-50", "1e-40",
        "0e999999", "0e-999999", "1e-99999999999999999999", "1e99999999999999999999",
        "16777216", "16777217", "16777218", "16777219", "33554433", "33554435",
        "0.1", "0.2", "0.3", "1.1", "3.14159265358979323846264338327950288", "2.5e-3",
        "123456789012345678901234567890", "0.000000000000000000000000000000000000000001",
        "1e-0000000000000000000000000000000000000000000050",
    };
    for (const char* s : fixed) check_float(s);
    check_float(std::string("1") + std::string(400, '0') + "e-400");
    check_float(std::string("0.") + std::string(400, '0') + "1e400");
    check_float(std::string("1.5\0" "7", 5));
    check_float(std::string("\0" "5", 2));
    check_float(std::string("0x\0" "1", 4));
    check_float(std::string("nan(\0)", 6));

    const char* ints[] = {"", " ", "+", "-", "0", "-0", "+0", "12", "-12", " 12 ", "12abc",
                          "2147483647", "2147483648", "-2147483648", "-2147483649",
                          "99999999999999999999", "-99999999999999999999", "0000000000000000000000012",
                          "1.5", "\v5", "\f-5", "0x10", "1e3", "+-1", "--1", " - 1"};
    for (const char* s : ints) check_int(s);
    check_int(std::string("1\0" "2", 3));

    // 2. every boundary float and its neighbourhood
    const uint32_t specials[] = {0x00000001, 0x00000002, 0x00000003, 0x000fffff, 0x00400000,
                                 0x007ffffe, 0x007fffff, 0x00800000, 0x00800001, 0x00ffffff,
                                 0x01000000, 0x3f800000, 0x3f7fffff, 0x4b7fffff, 0x4b800000,
                                 0x4b800001, 0x7f7ffffe, 0x7f7fffff, 0x7f000000};
    for (uint32_t u : specials) {
        around(u2f(u), rng);
        around(-u2f(u), rng);
    }

    // 3. random floats across the whole range, and random decimal strings
    for (long i = 0; i < n_random; ++i) {
        const uint32_t u = uint32_t(rng());
        const float x = u2f(u & 0x7fffffffu);
        if (i % 8 == 0) around(x, rng);
        else check_float(fmti("%.*g", int(rng() % 12 + 1), double(x)));
        // random digit strings with a point and an exponent
        std::string s;
        if (rng() % 4 == 0) s += (rng() & 1) ? "-" : "+";
        const int nd = int(rng() % 40) + 1;
        std::string dg = rand_digits(rng, nd);
        if (rng() % 3 == 0) dg = std::string(size_t(rng() % 6), '0') + dg;
        const size_t pt = size_t(rng() % (dg.size() + 1));
        if (rng() % 4 != 0) dg.insert(pt, ".");
        s += dg;
        if (rng() % 2) s += "e" + std::to_string(int(rng() % 110) - 60);
        check_float(s);
        // random hex
        std::string h = "0x" + std::string(size_t(rng() % 3), '0');
        const int nh = int(rng() % 24) + 1;
        static const char* hexd = "0123456789abcdefABCDEF";
        for (int k = 0; k < nh; ++k) h.push_back(hexd[rng() % 22]);
        if (rng() % 2) h.insert(2 + size_t(rng() % (h.size() - 1)), ".");
        h += "p" + std::to_string(int(rng() % 320) - 200);
        check_float(h);
        // random integers
        check_int(std::to_string(int64_t(rng() % 6000000000ull) - 3000000000ll));
        check_int(rand_digits(rng, int(rng() % 25) + 1));
    }
    // 4. the subnormal and tininess ranges, densely
    for (long i = 0; i < n_random / 4; ++i) {
        const uint32_t u = uint32_t(rng() % 0x01000000u);
        around(u2f(u), rng);
        // hexadecimal significands of 20-40 bits landing in every subnormal binade
        const int nbits = 20 + int(rng() % 21);
        const uint64_t m = (rng() & ((uint64_t(1) << (nbits - 1)) - 1)) | (uint64_t(1) << (nbits - 1));
        const int binade = -151 + int(rng() % 27);  // leading bit's exponent
        char buf[64];
        std::snprintf(buf, sizeof buf, "0x%" PRIx64 "p%d", m, binade - (nbits - 1));
        check_float(buf);
        std::snprintf(buf, sizeof buf, "0x%" PRIx64 "0p%d", m, binade - (nbits - 1) - 4);
        check_float(buf);
    }
    std::printf("numparse: %ld conversions checked against glibc, %ld mismatches\n", g_checked,
                g_bad);
    return g_bad ? 1 : 0;
}
