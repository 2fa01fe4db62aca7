// Cubic angular invariants q123, q233, q134 (rune/mobius/descriptor.py:
// 107-196): fixed term lists over the moment components of orders L <= 4,
// shared by the host packing and the descriptor kernels, which unroll them
// at compile time so every component index is a constant (the moments and
// the gradient accumulators stay in registers).
#pragma once

#include <utility>

namespace rune {

struct CubicTerm {
    int coef, sign, a, b, c;
};
// Cubic invariant term lists (coefficient index into C4B_123/233/134, sign,
// component indices), in the order of rune/mobius/descriptor.py:141-196.
inline constexpr CubicTerm kQ123[] = {
    {6, 1, 12, 2, 4}, {6, -1, 11, 2, 5}, {6, 1, 1, 11, 4}, {6, 1, 1, 12, 5}, {5, 1, 0, 11, 6},
    {5, 1, 0, 12, 7}, {3, 1, 14, 2, 6}, {3, -1, 13, 2, 7}, {3, 1, 1, 13, 6}, {3, 1, 1, 14, 7},
    {4, 1, 10, 0, 5}, {4, 1, 0, 4, 9},  {1, 1, 10, 2, 3}, {1, 1, 0, 3, 8},  {1, 1, 1, 3, 9},
    {0, 1, 10, 2, 6}, {0, -1, 10, 1, 7}, {0, -1, 2, 7, 9}, {0, -1, 1, 6, 9}, {2, -1, 2, 5, 8},
    {2, -1, 1, 4, 8}};
inline constexpr CubicTerm kQ233[] = {
    {0, 1, 3, 8, 8},    {1, 1, 10, 10, 3},  {1, 1, 3, 9, 9},    {2, -1, 10, 10, 6},
    {2, 1, 6, 9, 9},    {3, 1, 4, 8, 9},    {3, 1, 10, 5, 8},   {4, -1, 13, 13, 3},
    {4, -1, 14, 14, 3}, {5, -1, 14, 7, 9},  {5, -1, 13, 6, 9},  {5, -1, 10, 14, 6},
    {5, 1, 10, 13, 7},  {6, 1, 10, 7, 9},   {7, -1, 11, 6, 8},  {7, -1, 12, 7, 8},
    {8, 1, 11, 4, 9},   {8, 1, 12, 5, 9},   {8, 1, 10, 12, 4},  {8, -1, 10, 11, 5},
    {9, 1, 12, 14, 4},  {9, 1, 11, 14, 5},  {9, 1, 13, 11, 4},  {9, -1, 13, 12, 5}};
inline constexpr CubicTerm kQ134[] = {
    {0, -1, 10, 15, 2}, {0, -1, 1, 15, 9},  {1, 1, 0, 15, 8},   {2, -1, 1, 13, 18},
    {2, -1, 1, 14, 19}, {2, -1, 2, 14, 18}, {2, 1, 2, 13, 19},  {3, -1, 10, 18, 2},
    {3, 1, 1, 10, 19},  {3, 1, 1, 18, 9},   {3, 1, 2, 19, 9},   {4, 1, 1, 16, 8},
    {4, 1, 2, 17, 8},   {5, 1, 0, 10, 17},  {5, 1, 0, 16, 9},   {5, -1, 1, 11, 16},
    {5, -1, 1, 12, 17}, {5, -1, 2, 12, 16}, {5, 1, 2, 11, 17},  {6, 1, 1, 13, 22},
    {6, 1, 1, 14, 23},  {6, -1, 2, 14, 22}, {6, 1, 2, 13, 23},  {7, 1, 0, 11, 18},
    {7, 1, 0, 12, 19},  {8, 1, 0, 13, 20},  {8, 1, 0, 14, 21},  {9, 1, 1, 11, 20},
    {9, 1, 1, 12, 21},  {9, -1, 2, 12, 20}, {9, 1, 2, 11, 21}};
// C4B_123 / C4B_233 / C4B_134 (rune/mobius/descriptor.py:107-139).
inline constexpr double kC123[] = {-0.008418146349617, -0.016836292699234, -0.033672585398469,
                        -0.042090731748086, -0.067345170796937, -0.084181463496172,
                        -0.168362926992344};
inline constexpr double kC233[] = {0.008572620635186, 0.009644198214584, 0.019288396429168,
                        0.025717861905558, 0.026789439484956, 0.032147327381947,
                        0.038576792858337, 0.128589309527790, 0.192883964291685,
                        0.321473273819474};
inline constexpr double kC134[] = {0.003645164295772, 0.004860219061029, 0.006075273826286,
                        0.018225821478859, 0.024301095305146, 0.036451642957719,
                        0.042526916784005, 0.072903285915437, 0.085053833568010,
                        0.255161500704030};

// Components the cubic invariants involve (orders L <= 4).
constexpr int kCubicComps = 24;

template <size_t N>
constexpr bool cubic_in_range(const CubicTerm (&list)[N]) {
    for (size_t k = 0; k < N; ++k)
        if (list[k].a >= kCubicComps || list[k].b >= kCubicComps || list[k].c >= kCubicComps)
            return false;
    return true;
}
static_assert(cubic_in_range(kQ123) && cubic_in_range(kQ233) && cubic_in_range(kQ134),
              "cubic invariant component beyond kCubicComps");

template <int W>
struct CubicList;
template <>
struct CubicList<0> {
    static constexpr const CubicTerm *terms = kQ123;
    static constexpr const double *coef = kC123;
    static constexpr int n = int(sizeof(kQ123) / sizeof(CubicTerm));
};
template <>
struct CubicList<1> {
    static constexpr const CubicTerm *terms = kQ233;
    static constexpr const double *coef = kC233;
    static constexpr int n = int(sizeof(kQ233) / sizeof(CubicTerm));
};
template <>
struct CubicList<2> {
    static constexpr const CubicTerm *terms = kQ134;
    static constexpr const double *coef = kC134;
    static constexpr int n = int(sizeof(kQ134) / sizeof(CubicTerm));
};

// Signed coefficient of term K of invariant W, rounded to fp32 as the packed
// tables hold it.
template <int W, int K>
constexpr float cubic_coef() {
    return float(double(CubicList<W>::terms[K].sign) *
                 CubicList<W>::coef[CubicList<W>::terms[K].coef]);
}

template <int W, int K>
__device__ inline void cubic_term(const float (&s)[kCubicComps], float &r) {
    constexpr CubicTerm t = CubicList<W>::terms[K];
    r = r + cubic_coef<W, K>() * ((s[t.a] * s[t.b]) * s[t.c]);
}

// Invariant W of one channel's moments s, terms summed in list order.
template <int W, size_t... K>
__device__ inline float cubic_value(const float (&s)[kCubicComps], std::index_sequence<K...>) {
    float r = 0.0f;
    (cubic_term<W, int(K)>(s, r), ...);
    return r;
}
template <int W>
__device__ inline float cubic_value(const float (&s)[kCubicComps]) {
    return cubic_value<W>(s, std::make_index_sequence<CubicList<W>::n>{});
}

template <int W, int K>
__device__ inline void cubic_grad_term(const float (&s)[kCubicComps], float g, float *w, int nlm) {
    constexpr CubicTerm t = CubicList<W>::terms[K];
    const float gc = g * cubic_coef<W, K>();
    if (t.a < nlm) w[t.a] += gc * (s[t.b] * s[t.c]);
    if (t.b < nlm) w[t.b] += gc * (s[t.a] * s[t.c]);
    if (t.c < nlm) w[t.c] += gc * (s[t.a] * s[t.b]);
}

// w[c] += g * d(invariant W)/ds_c for c < nlm, terms in list order (w: one
// channel's gradient row, every index a constant offset).
template <int W, size_t... K>
__device__ inline void cubic_grad(const float (&s)[kCubicComps], float g, float *w, int nlm,
                                  std::index_sequence<K...>) {
    (cubic_grad_term<W, int(K)>(s, g, w, nlm), ...);
}
template <int W>
__device__ inline void cubic_grad(const float (&s)[kCubicComps], float g, float *w, int nlm) {
    cubic_grad<W>(s, g, w, nlm, std::make_index_sequence<CubicList<W>::n>{});
}

}  // namespace rune
