// numparse_table.hpp -- host-side construction of the power-of-ten table used
// by numparse.hpp: for q in [kPow10Min, kPow10Max], 10^q bracketed as
// [mant, mant + 1) * 2^exp2 with a normalised 64-bit mant.  Computed exactly
// with a small big integer (no floating point involved).
#pragma once

#include <cstdint>
#include <vector>

#include "numparse.hpp"

namespace tg {
namespace numparse {

namespace detail {

using Limbs = std::vector<uint32_t>;  // little endian, no leading zero limbs

inline void trim(Limbs& a) {
    while (!a.empty() && a.back() == 0) a.pop_back();
}
inline int bit_length(const Limbs& a) {
    if (a.empty()) return 0;
    return int(a.size() - 1) * 32 + (32 - __builtin_clz(a.back()));
}
inline bool bit(const Limbs& a, int i) {
    const size_t l = size_t(i) / 32;
    return l < a.size() && ((a[l] >> (i % 32)) & 1u);
}
inline void mul_small(Limbs& a, uint32_t m) {
    uint64_t carry = 0;
    for (auto& d : a) {
        const uint64_t t = uint64_t(d) * m + carry;
        d = uint32_t(t);
        carry = t >> 32;
    }
    if (carry) a.push_back(uint32_t(carry));
}
inline int cmp(const Limbs& a, const Limbs& b) {
    if (a.size() != b.size()) return a.size() < b.size() ? -1 : 1;
    for (size_t i = a.size(); i-- > 0;)
        if (a[i] != b[i]) return a[i] < b[i] ? -1 : 1;
    return 0;
}
inline void sub(Limbs& a, const Limbs& b) {  // a -= b, a >= b
    int64_t borrow = 0;
    for (size_t i = 0; i < a.size(); ++i) {
        int64_t t = int64_t(a[i]) - borrow - (i < b.size() ? int64_t(b[i]) : 0);
        borrow = t < 0;
        if (t < 0) t += int64_t(1) << 32;
        a[i] = uint32_t(t);
    }
    trim(a);
}
inline void shl1_add(Limbs& a, bool b) {  // a = 2a + b
    uint32_t carry = b ? 1u : 0u;
    for (auto& d : a) {
        const uint32_t nc = d >> 31;
        d = (d << 1) | carry;
        carry = nc;
    }
    if (carry) a.push_back(carry);
}

}  // namespace detail

/// Fills out[kPow10Count] (index q - kPow10Min).
inline void build_pow10_table(Pow10Entry* out) {
    using namespace detail;
    for (int q = kPow10Min; q <= kPow10Max; ++q) {
        Limbs p{1};
        for (int i = 0; i < (q < 0 ? -q : q); ++i) mul_small(p, 10u);
        Pow10Entry& t = out[q - kPow10Min];
        const int L = bit_length(p);
        if (q >= 0) {
            uint64_t m = 0;
            bool exact = true;
            for (int i = 0; i < 64; ++i) {  // the top 64 bits (zero-extended below)
                const int src = L - 1 - i;
                m = (m << 1) | (src >= 0 && bit(p, src) ? 1u : 0u);
            }
            for (int i = 0; i < L - 64; ++i) exact &= !bit(p, i);
            t.mant = m;
            t.exp2 = L - 64;
            t.exact = exact ? 1 : 0;
        } else {
            // floor(2^(63 + L) / 10^-q): restoring division, one quotient bit
            // per numerator bit (the numerator is a single 1 bit)
            const int nbits = 63 + L;
            Limbs rem;
            uint64_t quo = 0;
            for (int i = nbits; i >= 0; --i) {
                shl1_add(rem, i == nbits);
                trim(rem);
                const bool ge = cmp(rem, p) >= 0;
                if (ge) sub(rem, p);
                quo = (quo << 1) | (ge ? 1u : 0u);
            }
            t.mant = quo;
            t.exp2 = -nbits;
            t.exact = 0;
        }
    }
}

}  // namespace numparse
}  // namespace tg
