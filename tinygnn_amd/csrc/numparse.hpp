// numparse.hpp -- the number conversions behind TinyGNN's CSV readers, for
// host and device code.
//
// The reference parses CSV fields with std::stoi (node ids, edge endpoints;
// graph_loader.cpp:81-82,111) and std::stof (features, :134).  libstdc++
// implements them as strtol(s, &end, 10) / strtof(s, &end) on the field's
// C string, throwing std::invalid_argument when nothing converts and
// std::out_of_range when errno is ERANGE (or, for stoi, when the long does
// not fit an int).  Characters after the converted prefix are ignored.
// These functions restate that contract on a byte range [p, e):
//
//   parse_int   -> kOk / kInvalid / kRange, the int value;
//   parse_float -> kOk / kInvalid / kRange, the IEEE binary32 bits that
//                  glibc's strtof returns (round to nearest even), with
//                  kRange exactly where glibc sets ERANGE:
//                    * overflow to infinity;
//                    * underflow: the result is tiny (below 2^-126 after
//                      rounding to 24 bits with an unbounded exponent) and
//                      inexact;
//                    * a NaN payload "nan(n-char-sequence)" whose strtoull
//                      (base 0) conversion overflows.
//
// Accepted syntax (C11 7.22.1.3): optional white space (' ', \t \n \v \f
// \r), an optional sign, then a decimal significand with an optional
// exponent, "0x" and a hexadecimal significand with an optional binary
// exponent, "inf"/"infinity", or "nan"/"nan(n-char-sequence)", all letters
// case-insensitive.  A NUL byte ends the field, as it ends the C string the
// reference hands to strtof.
//
// Decimal conversion is exact.  The first 19 significant digits w, a sticky
// flag for the rest, and the power q of ten give V = w * 10^q.  The 128-bit
// product of w with a 64-bit truncation of 10^q (a table computed exactly by
// the host) brackets V in [P, P + E].  Rounding is decided from P unless a
// rounding midpoint, a representable value (for the underflow flag) or the
// tininess boundary lies inside the bracket.  Only then is V compared
// exactly with that threshold: the threshold's decimal expansion is
// generated in a small big integer and compared digit by digit with the
// field's own digits.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define TG_HD __host__ __device__ inline
#define TG_HD_COLD __host__ __device__ __attribute__((noinline))
#else
#define TG_HD inline
#define TG_HD_COLD inline
#endif

namespace tg {
namespace numparse {

enum : int { kOk = 0, kInvalid = 1, kRange = 2 };

typedef unsigned __int128 u128;

// 10^q in [mant, mant + 1) * 2^exp2, mant normalised (bit 63 set); exact
// when 10^q == mant * 2^exp2.
struct Pow10Entry {
    uint64_t mant;
    int32_t exp2;
    int32_t exact;
};
constexpr int kPow10Min = -70;
constexpr int kPow10Max = 40;
constexpr int kPow10Count = kPow10Max - kPow10Min + 1;

TG_HD bool is_space(unsigned c) { return c == ' ' || (c >= 9 && c <= 13); }
TG_HD bool is_digit(unsigned c) { return c - '0' < 10u; }
TG_HD bool is_alpha(unsigned c) { return ((c | 0x20u) - 'a') < 26u; }
TG_HD int hex_val(unsigned c) {
    if (c - '0' < 10u) return int(c - '0');
    c |= 0x20u;
    if (c - 'a' < 6u) return int(c - 'a') + 10;
    return -1;
}
TG_HD unsigned lower(unsigned c) { return c | 0x20u; }

// std::stoi: strtol(s, &end, 10), then the int range check.
TG_HD int parse_int(const unsigned char* p, const unsigned char* e, int32_t* out) {
    while (p < e && is_space(*p)) ++p;
    bool neg = false;
    if (p < e && (*p == '+' || *p == '-')) {
        neg = *p == '-';
        ++p;
    }
    if (p >= e || !is_digit(*p)) return kInvalid;
    uint64_t v = 0;
    bool big = false;
    for (; p < e && is_digit(*p); ++p) {
        if (!big) {
            v = v * 10u + (*p - '0');
            big = v > 0x80000000ull;
        }
    }
    if (big || (!neg && v > 0x7fffffffull)) return kRange;
    *out = neg ? int32_t(uint32_t(0u - uint32_t(v))) : int32_t(v);
    return kOk;
}

// ---------------------------------------------------------------------------
// Exact comparison of a decimal significand with a dyadic threshold.

// Little-endian base-2^32 big integer, enough for Tm * 5^151 with Tm < 2^32.
struct Big {
    static constexpr int kLimbs = 14;
    uint32_t d[kLimbs];
    int n;
};

TG_HD void big_set(Big& b, uint64_t v) {
    b.d[0] = uint32_t(v);
    b.d[1] = uint32_t(v >> 32);
    b.n = b.d[1] ? 2 : (b.d[0] ? 1 : 0);
}
TG_HD void big_mul_small(Big& b, uint32_t m) {
    uint64_t carry = 0;
    for (int i = 0; i < b.n; ++i) {
        const uint64_t t = uint64_t(b.d[i]) * m + carry;
        b.d[i] = uint32_t(t);
        carry = t >> 32;
    }
    if (carry && b.n < Big::kLimbs) b.d[b.n++] = uint32_t(carry);
}
TG_HD void big_shl(Big& b, int s) {
    const int limbs = s / 32, bits = s % 32;
    if (b.n == 0) return;
    int n = b.n + limbs + 1;
    if (n > Big::kLimbs) n = Big::kLimbs;
    for (int i = n - 1; i >= 0; --i) {
        const int src = i - limbs;
        uint32_t hi = (src >= 0 && src < b.n) ? b.d[src] : 0u;
        uint32_t lo = (src - 1 >= 0 && src - 1 < b.n) ? b.d[src - 1] : 0u;
        b.d[i] = bits ? (hi << bits) | (lo >> (32 - bits)) : hi;
    }
    b.n = n;
    while (b.n > 0 && b.d[b.n - 1] == 0) --b.n;
}
// b /= 1e9, returns the remainder.
TG_HD uint32_t big_div_1e9(Big& b) {
    uint64_t rem = 0;
    for (int i = b.n - 1; i >= 0; --i) {
        const uint64_t cur = (rem << 32) | b.d[i];
        b.d[i] = uint32_t(cur / 1000000000u);
        rem = cur % 1000000000u;
    }
    while (b.n > 0 && b.d[b.n - 1] == 0) --b.n;
    return uint32_t(rem);
}

// Iterates the significant digits of a decimal significand [p, e) (digits
// and at most one '.'), starting at the first non-zero digit.
struct DigitIter {
    const unsigned char* p;
    const unsigned char* e;
    TG_HD int next() {  // the next digit, or -1 at the end
        while (p < e) {
            const unsigned c = *p++;
            if (c == '.') continue;
            return int(c - '0');
        }
        return -1;
    }
};

// sign(V - Tm * 2^t2), V = 0.d1 d2 ... * 10^ed with d1 != 0 (the digits in
// [mb, me) after their leading zeros), Tm > 0.
// Kept out of line on the device: it runs for a tiny fraction of fields and
// would otherwise hold its big integers in the caller's registers.
TG_HD_COLD int cmp_exact(const unsigned char* mb, const unsigned char* me, int64_t ed, uint64_t tm,
                    int t2) {
    Big b;
    big_set(b, tm);
    int et = 0;
    if (t2 >= 0) {
        big_shl(b, t2);
    } else {
        for (int i = 0; i < -t2; ++i) big_mul_small(b, 5u);
        et = t2;
    }
    // base-1e9 chunks, least significant first
    uint32_t ch[16];
    int nch = 0;
    while (b.n > 0 && nch < 16) ch[nch++] = big_div_1e9(b);
    int top_digits = 0;
    for (uint32_t t = ch[nch - 1]; t; t /= 10u) ++top_digits;
    const int64_t nt = int64_t(nch - 1) * 9 + top_digits;
    const int64_t er = nt + et;
    if (ed != er) return ed > er ? 1 : -1;
    // skip the field's leading zeros
    DigitIter it{mb, me};
    int dv = it.next();
    while (dv == 0) dv = it.next();
    // threshold digits, most significant first
    uint32_t pw = 1;
    for (int i = 1; i < top_digits; ++i) pw *= 10u;
    int ci = nch - 1;
    uint32_t cur = ch[ci];
    while (true) {
        int dt = -1;
        if (ci >= 0) {
            dt = int(cur / pw);
            cur %= pw;
            if (pw == 1) {
                --ci;
                if (ci >= 0) {
                    cur = ch[ci];
                    pw = 100000000u;
                }
            } else {
                pw /= 10u;
            }
        }
        if (dv < 0 && dt < 0) return 0;
        const int a = dv < 0 ? 0 : dv;
        const int t = dt < 0 ? 0 : dt;
        if (a != t) return a > t ? 1 : -1;
        if (dt < 0) {  // threshold exhausted: V is larger iff a non-zero digit remains
            for (dv = it.next(); dv >= 0; dv = it.next())
                if (dv) return 1;
            return 0;
        }
        dv = dv < 0 ? -1 : it.next();
    }
}

// ---------------------------------------------------------------------------
// Rounding V = (P + delta) * 2^x to binary32.
//
// P has bit 127 set.  The uncertainty model:
//   kExact:    delta = 0;
//   kSticky:   0 < delta < 2^s, every threshold a multiple of 2^s (hex);
//   kInterval: 0 <= delta <= E; a threshold inside [P, P + E] is compared
//              exactly with the decimal digits (cmp_exact).
enum : int { kExact = 0, kSticky = 1, kInterval = 2 };

struct RoundCtx {
    u128 P, E;
    int x;
    int kind;
    // decimal digits for the exact comparison
    const unsigned char* mb;
    const unsigned char* me;
    int64_t ed;
};

TG_HD int ctz128(u128 v) {
    const uint64_t lo = uint64_t(v);
    return lo ? __builtin_ctzll(lo) : 64 + __builtin_ctzll(uint64_t(v >> 64));
}

// sign(V - T * 2^x); T given as a u128, or 2^128 when top is set.
TG_HD int cmp_v(const RoundCtx& c, u128 t, bool top) {
    if (c.kind == kExact) {
        if (top) return -1;
        return c.P > t ? 1 : (c.P < t ? -1 : 0);
    }
    if (c.kind == kSticky) {
        if (top) return -1;
        return c.P >= t ? 1 : -1;
    }
    if (!top && c.P > t) return 1;
    const u128 hi = c.P + c.E;
    const bool hi_overflow = hi < c.P;
    if (!top && !hi_overflow && hi < t) return -1;
    if (top && !hi_overflow) return -1;
    // the threshold lies in [P, P + E]: exact comparison
    int tz;
    uint64_t tm;
    if (top) {
        tz = 128;
        tm = 1;
    } else {
        tz = ctz128(t);
        tm = uint64_t(t >> tz);
    }
    return cmp_exact(c.mb, c.me, c.ed, tm, tz + c.x);
}

// tiny_c, when given, is the value used for the tininess decision (see
// parse_hex); otherwise c.
TG_HD int round_to_f32(const RoundCtx& c, uint32_t sign, uint32_t* out,
                       const RoundCtx* tiny_c = nullptr) {
    const int e = 127 + c.x;  // P * 2^x in [2^e, 2^(e+1))
    if (e > 127) {
        *out = sign | 0x7f800000u;
        return kRange;
    }
    const int cut = e >= -126 ? 104 : 104 + (-126 - e);
    if (cut > 128) {
        // P * 2^x < 2^-150.  Below 2^-150 (or at it: a tie, to even) V rounds
        // to zero; V reaches past 2^-150 only from e = -151 and then rounds to
        // the smallest subnormal.  Inexact either way.
        const bool above = e == -151 && cmp_v(c, 0, true) > 0;
        *out = sign | (above ? 1u : 0u);
        return kRange;
    }
    const u128 one = 1;
    const u128 kept = cut == 128 ? u128(0) : (c.P >> cut);
    const u128 g0 = cut == 128 ? u128(0) : (kept << cut);
    const u128 mid = g0 + (one << (cut - 1));
    const int r = cmp_v(c, mid, false);
    const bool up = r > 0 || (r == 0 && (uint64_t(kept) & 1u));
    const uint64_t R = uint64_t(kept) + (up ? 1u : 0u);
    if (e >= -126) {
        int be = e + 127;
        uint64_t m = R;
        if (m >> 24) {
            m >>= 1;
            ++be;
        }
        if (be >= 255) {
            *out = sign | 0x7f800000u;
            return kRange;
        }
        *out = sign | (uint32_t(be) << 23) | (uint32_t(m) & 0x7fffffu);
        return kOk;
    }
    *out = sign | uint32_t(R);  // subnormal (R == 2^23 encodes FLT_MIN)
    bool tiny = true;
    if (e == -127) {  // tininess after rounding to 24 bits
        const RoundCtx& tc = tiny_c ? *tiny_c : c;
        const u128 k24 = tc.P >> 104;
        if (uint64_t(k24) == 0xffffffu) {
            const int r2 = cmp_v(tc, (k24 << 104) + (one << 103), false);
            tiny = !(r2 > 0 || r2 == 0);  // k24 is odd: a tie rounds up
        }
    }
    if (!tiny) return kOk;
    // inexact unless V is the grid point it rounds to
    bool exact;
    if (!up) {
        exact = cmp_v(c, g0, false) == 0;
    } else {
        const u128 g1 = kept + 1;
        const bool top = cut == 128 ? true : ((g1 << cut) >> cut) != g1;
        exact = cmp_v(c, top ? u128(0) : (g1 << cut), top) == 0;
    }
    return exact ? kOk : kRange;
}

// ---------------------------------------------------------------------------

// strtoull(s, &end, 0) over an n-char-sequence [s, r): sets *val, returns the
// end of the conversion; *overflow when the value exceeds 2^64 - 1.
TG_HD const unsigned char* strtoull0(const unsigned char* s, const unsigned char* r, uint64_t* val,
                                     bool* overflow) {
    unsigned base = 10;
    const unsigned char* q = s;
    if (q < r && *q == '0') {
        if (q + 2 < r && lower(q[1]) == 'x' && hex_val(q[2]) >= 0) {
            base = 16;
            q += 2;
        } else {
            base = 8;
        }
    }
    uint64_t v = 0;
    bool of = false;
    const unsigned char* start = q;
    for (; q < r; ++q) {
        const int dv = hex_val(*q);
        if (dv < 0 || unsigned(dv) >= base) break;
        if (!of) {
            const u128 t = u128(v) * base + unsigned(dv);
            if (t >> 64) {
                of = true;
                v = ~uint64_t(0);
            } else {
                v = uint64_t(t);
            }
        }
    }
    *val = v;
    *overflow = of;
    return q == start ? s : q;
}

TG_HD int parse_hex(const unsigned char* p, const unsigned char* e, uint32_t sign, uint32_t* out) {
    uint64_t m = 0;
    int nd = 0;
    bool sticky = false, point = false, started = false;
    int64_t e2 = 0;
    for (; p < e; ++p) {
        const unsigned c = *p;
        if (c == '.') {
            if (point) break;
            point = true;
            continue;
        }
        const int v = hex_val(c);
        if (v < 0) break;
        if (!started && v == 0) {
            if (point) e2 -= 4;
            continue;
        }
        started = true;
        if (nd < 16) {
            m = (m << 4) | unsigned(v);
            ++nd;
            if (point) e2 -= 4;
        } else {
            sticky |= v != 0;
            if (!point) e2 += 4;
        }
    }
    if (p < e && lower(*p) == 'p') {
        const unsigned char* q = p + 1;
        bool neg = false;
        if (q < e && (*q == '+' || *q == '-')) {
            neg = *q == '-';
            ++q;
        }
        if (q < e && is_digit(*q)) {
            int64_t ex = 0;
            for (; q < e && is_digit(*q); ++q)
                if (ex < 100000000) ex = ex * 10 + (*q - '0');
            e2 += neg ? -ex : ex;
        }
    }
    if (!started) {
        *out = sign;
        return kOk;
    }
    const int lz = __builtin_clzll(m);
    const uint64_t wn = m << lz;
    RoundCtx c;
    c.P = u128(wn) << 64;
    c.E = 0;
    const int64_t x = e2 - lz - 64;
    if (x > 1000) {
        *out = sign | 0x7f800000u;
        return kRange;
    }
    if (x < -1000) {
        *out = sign;
        return kRange;
    }
    c.x = int(x);
    c.kind = sticky ? kSticky : kExact;
    c.mb = c.me = nullptr;
    c.ed = 0;
    if (127 + c.x < -126) {
        // A subnormal result.  glibc's hexadecimal conversion rounds it
        // without the 25th significant bit of the digits (the first bit past
        // a 24-bit significand): that bit counts neither as the rounding bit
        // nor as a sticky bit, nor for ERANGE.  It still counts for the
        // tininess decision.  Reproduced here because the reference reads
        // its features through that function; measured against glibc 2.35
        // (tests/cpp/test_numparse.cpp).
        RoundCtx g = c;
        g.P = u128(wn & ~(uint64_t(1) << 39)) << 64;
        return round_to_f32(g, sign, out, &c);
    }
    return round_to_f32(c, sign, out);
}

TG_HD int parse_dec(const unsigned char* p, const unsigned char* e, uint32_t sign,
                    const Pow10Entry* tab, uint32_t* out) {
    const unsigned char* mb = p;
    uint64_t w = 0;
    int nd = 0;
    bool sticky = false, point = false, any = false, started = false;
    int64_t e10 = 0;
    for (; p < e; ++p) {
        const unsigned c = *p;
        if (c == '.') {
            if (point) break;
            point = true;
            continue;
        }
        if (!is_digit(c)) break;
        any = true;
        const unsigned v = c - '0';
        if (!started && v == 0) {
            if (point) --e10;
            continue;
        }
        started = true;
        if (nd < 19) {
            w = w * 10u + v;
            ++nd;
            if (point) --e10;
        } else {
            sticky |= v != 0;
            if (!point) ++e10;
        }
    }
    if (!any) return kInvalid;
    const unsigned char* me = p;
    if (p < e && lower(*p) == 'e') {
        const unsigned char* q = p + 1;
        bool neg = false;
        if (q < e && (*q == '+' || *q == '-')) {
            neg = *q == '-';
            ++q;
        }
        if (q < e && is_digit(*q)) {
            int64_t ex = 0;
            for (; q < e && is_digit(*q); ++q)
                if (ex < 100000000) ex = ex * 10 + (*q - '0');
            e10 += neg ? -ex : ex;
        }
    }
    if (!started) {
        *out = sign;
        return kOk;
    }
    const int64_t ed = e10 + nd;  // V in [10^(ed-1), 10^ed)
    if (ed - 1 >= 39) {
        *out = sign | 0x7f800000u;
        return kRange;
    }
    if (ed <= -46) {
        *out = sign;
        return kRange;
    }
    const Pow10Entry t = tab[int(e10) - kPow10Min];
    const int lz = __builtin_clzll(w);
    const uint64_t wn = w << lz;
    RoundCtx c;
    c.P = u128(wn) * t.mant;
    c.E = (t.exact ? u128(0) : u128(wn)) + (sticky ? (u128(t.mant) + 1) << lz : u128(0));
    int x = t.exp2 - lz;
    if (!(c.P >> 127)) {
        c.P <<= 1;
        c.E <<= 1;
        --x;
    }
    c.x = x;
    c.kind = c.E == 0 ? kExact : kInterval;
    c.mb = mb;
    c.me = me;
    c.ed = ed;
    return round_to_f32(c, sign, out);
}

// std::stof on [p, e): glibc strtof's value and ERANGE, as described above.
TG_HD int parse_float(const unsigned char* p, const unsigned char* e, const Pow10Entry* tab,
                      uint32_t* out) {
    while (p < e && is_space(*p)) ++p;
    uint32_t sign = 0;
    if (p < e && (*p == '+' || *p == '-')) {
        sign = *p == '-' ? 0x80000000u : 0u;
        ++p;
    }
    if (p >= e) return kInvalid;
    const unsigned c = *p;
    if (c == '0' && p + 1 < e && lower(p[1]) == 'x') {
        const unsigned char* h = p + 2;
        const bool digits = (h < e && hex_val(*h) >= 0) ||
                            (h + 1 < e && *h == '.' && hex_val(h[1]) >= 0);
        if (digits) return parse_hex(h, e, sign, out);
        *out = sign;  // "0x" without a hex digit converts as "0"
        return kOk;
    }
    if (lower(c) == 'i') {
        if (e - p >= 3 && lower(p[1]) == 'n' && lower(p[2]) == 'f') {
            *out = sign | 0x7f800000u;
            return kOk;
        }
        return kInvalid;
    }
    if (lower(c) == 'n') {
        if (!(e - p >= 3 && lower(p[1]) == 'a' && lower(p[2]) == 'n')) return kInvalid;
        uint32_t payload = 0;
        int st = kOk;
        const unsigned char* q = p + 3;
        if (q < e && *q == '(') {
            const unsigned char* s = q + 1;
            const unsigned char* r = s;
            while (r < e && (is_digit(*r) || is_alpha(*r) || *r == '_')) ++r;
            if (r < e && *r == ')') {
                uint64_t v;
                bool of;
                const unsigned char* end = strtoull0(s, r, &v, &of);
                if (of) st = kRange;
                if (end == r) payload = uint32_t(v) & 0x3fffffu;
            }
        }
        *out = sign | 0x7fc00000u | payload;
        return st;
    }
    return parse_dec(p, e, sign, tab, out);
}

}  // namespace numparse
}  // namespace tg
