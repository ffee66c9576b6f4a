// gqa_device.h -- device helpers shared by the gfx950 kernels (wave64, CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gqa {

constexpr int kHq = 32;       // Q heads
constexpr int kHkv = 8;       // KV heads
constexpr int kGroup = 4;     // Q heads per KV head
constexpr int kD = 128;       // head_dim
constexpr int kWave = 64;
constexpr int kPairs = kD / 2;

// theta^(-2i/128) for i < 64, computed on the host in double exactly as the
// golden computes it (pyfiles/gen_gqa_wrapper_vectors.py:30).
struct RopeTable {
    double inv_freq[kPairs];
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Eight BF16 codes packed in a uint4 -> eight floats (element 0 in the low half
// of the first dword, i.e. memory order).
__device__ __forceinline__ void unpack8(const uint4& w, float (&f)[8]) {
    f[0] = bf16_lo(w.x); f[1] = bf16_hi(w.x);
    f[2] = bf16_lo(w.y); f[3] = bf16_hi(w.y);
    f[4] = bf16_lo(w.z); f[5] = bf16_hi(w.z);
    f[6] = bf16_lo(w.w); f[7] = bf16_hi(w.w);
}

// float -> BF16 code, round to nearest even (NaN -> quiet NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// An attention output element -> BF16 code: f32_to_bf16_rne, except that a NaN becomes
// 0xffc0.  The golden's f32_to_bf16 keeps a NaN's sign (pyfiles/gqa_reference.py:17-19),
// and on the x86 hosts the golden runs on, a NaN that an invalid operation creates
// (inf - inf, 0 * inf: the only way a row of finite or infinite inputs reaches NaN) is
// the default NaN, whose sign bit is set; every later operation passes it on.  (A NaN
// input in a key the row reads keeps its own sign in the golden; that is not followed.)
__device__ __forceinline__ uint16_t f32_to_bf16_out(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffc0;
    return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// double -> f32 (RNE) -> BF16 (RNE): the reference's f32_to_bf16 path
// (pyfiles/gqa_reference.py:15-19).
__device__ __forceinline__ uint16_t f64_to_bf16_via_f32(double d) {
    return f32_to_bf16_rne(static_cast<float>(d));
}

// Exponent of the exact weight 2^(m - m_ref) of a running max m against a reference
// m_ref >= m (both integer-valued floats, m_ref finite), clamped at -2048: every ldexp of a
// float or double by less gives 0, and converting a difference beyond the int range is
// undefined.  m = -inf gives -2048, weight 0.
__device__ __forceinline__ int max_shift(float m, float m_ref) {
    return static_cast<int>(fmaxf(m - m_ref, -2048.f));
}

// The same for running maxima kept in double (the fp64 paths: their scores may lie far
// beyond 2^24, where an integer-valued fp32 max could not sit within a few units of the
// largest score, and p of that key would underflow).
__device__ __forceinline__ int max_shift_f64(double m, double m_ref) {
    return static_cast<int>(fmax(m - m_ref, -2048.0));
}

// DPP lane moves (row = 16 lanes).  Control codes: quad_perm [1,0,3,2] = 0xB1,
// quad_perm [2,3,0,1] = 0x4E, quad_perm [h,h,h,h] = 0x55*h (broadcast lane h of each
// quad), row_ror:n = 0x120 + n.
template <int kCtrl>
__device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xf, 0xf, false));
}

template <int kCtrl>
__device__ __forceinline__ int dpp_i(int x) {
    return __builtin_amdgcn_update_dpp(0, x, kCtrl, 0xf, 0xf, false);
}

template <int kCtrl>
__device__ __forceinline__ double dpp_d(double x) {
    const unsigned long long u = static_cast<unsigned long long>(__double_as_longlong(x));
    const unsigned lo = static_cast<unsigned>(dpp_i<kCtrl>(static_cast<int>(u)));
    const unsigned hi = static_cast<unsigned>(dpp_i<kCtrl>(static_cast<int>(u >> 32)));
    return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}

// Sum over the 16 lanes of a DPP row; every lane of the row gets the total.
__device__ __forceinline__ float row16_sum(float x) {
    x += dpp_f<0xB1>(x);
    x += dpp_f<0x4E>(x);
    x += dpp_f<0x124>(x);
    x += dpp_f<0x128>(x);
    return x;
}

__device__ __forceinline__ float row16_max(float x) {
    x = fmaxf(x, dpp_f<0xB1>(x));
    x = fmaxf(x, dpp_f<0x4E>(x));
    x = fmaxf(x, dpp_f<0x124>(x));
    x = fmaxf(x, dpp_f<0x128>(x));
    return x;
}

// The same two reductions in double.
__device__ __forceinline__ double row16_sum_f64(double x) {
    x += dpp_d<0xB1>(x);
    x += dpp_d<0x4E>(x);
    x += dpp_d<0x124>(x);
    x += dpp_d<0x128>(x);
    return x;
}

__device__ __forceinline__ double row16_min_f64(double x) {
    x = fmin(x, dpp_d<0xB1>(x));
    x = fmin(x, dpp_d<0x4E>(x));
    x = fmin(x, dpp_d<0x124>(x));
    x = fmin(x, dpp_d<0x128>(x));
    return x;
}

// Across the four rows of a wave (lanes l, l^16, l^32, l^48).
__device__ __forceinline__ float cross_row_sum(float x) {
    x += __shfl_xor(x, 16);
    x += __shfl_xor(x, 32);
    return x;
}

__device__ __forceinline__ float cross_row_max(float x) {
    x = fmaxf(x, __shfl_xor(x, 16));
    x = fmaxf(x, __shfl_xor(x, 32));
    return x;
}

// x of lane l combined with x of lane l ^ 16 (row pairs 0-1, 2-3) or l ^ 32 (halves) through
// gfx950's lane swaps v_permlane16_swap_b32 / v_permlane32_swap_b32 (VALU, no LDS round
// trip).  A swap returns {own, partner} in an order fixed by the lane, and the two are
// combined commutatively, so both lanes of a pair get the same value, bit for bit the value
// that x + __shfl_xor(x, 16) (or 32) gives.  All 64 lanes must be active.
__device__ __forceinline__ float swap16_max(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float swap32_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

template <bool k32>
__device__ __forceinline__ double swap_add_f64(double x) {
    const unsigned long long u = static_cast<unsigned long long>(__double_as_longlong(x));
    const unsigned lo = static_cast<unsigned>(u), hi = static_cast<unsigned>(u >> 32);
    const auto rl = k32 ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false)
                        : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto rh = k32 ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false)
                        : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    const double a = __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(rh[0]) << 32) | rl[0]));
    const double b = __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(rh[1]) << 32) | rl[1]));
    return a + b;
}

// The larger of x in lane l and in lane l ^ 16 (k32: l ^ 32), as swap_add_f64.
template <bool k32>
__device__ __forceinline__ double swap_max_f64(double x) {
    const unsigned long long u = static_cast<unsigned long long>(__double_as_longlong(x));
    const unsigned lo = static_cast<unsigned>(u), hi = static_cast<unsigned>(u >> 32);
    const auto rl = k32 ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false)
                        : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto rh = k32 ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false)
                        : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    const double a = __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(rh[0]) << 32) | rl[0]));
    const double b = __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(rh[1]) << 32) | rl[1]));
    return fmax(a, b);
}

// Largest x over the wave (all 64 lanes active): within rows by DPP, across them by swaps.
__device__ __forceinline__ double wave_max_f64(double x) {
    x = fmax(x, dpp_d<0xB1>(x));
    x = fmax(x, dpp_d<0x4E>(x));
    x = fmax(x, dpp_d<0x124>(x));
    x = fmax(x, dpp_d<0x128>(x));
    return swap_max_f64<true>(swap_max_f64<false>(x));
}

// Per-half maxima of two pairs of 16-bit codes (v_pk_max_u16): for BF16 magnitudes (sign
// cleared) the larger code is the larger magnitude, NaN and infinity above every finite value.
__device__ __forceinline__ uint32_t pk_max_u16(uint32_t x, uint32_t y) {
    typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2_t, x),
                                                                  __builtin_bit_cast(u16x2_t, y)));
}

__device__ __forceinline__ uint32_t pk_min_u16(uint32_t x, uint32_t y) {
    typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(u16x2_t, x),
                                                                  __builtin_bit_cast(u16x2_t, y)));
}

// acc + the squares of the two BF16 values in w (v_dot2_f32_bf16, fp32 accumulation).
__device__ __forceinline__ float bf16x2_sq_acc(uint32_t w, float acc) {
    typedef __bf16 b16x2_t __attribute__((ext_vector_type(2)));
    const b16x2_t v = __builtin_bit_cast(b16x2_t, w);
    return __builtin_amdgcn_fdot2_f32_bf16(v, v, acc, false);
}

__device__ __forceinline__ float wave_sum(float x) { return cross_row_sum(row16_sum(x)); }
__device__ __forceinline__ float wave_max(float x) { return cross_row_max(row16_max(x)); }


// sin and cos of angle = position * inv_freq, in double.  The angle (up to ~2^31 rad)
// is first reduced modulo 2*pi with a two-part Cody-Waite constant and fused
// multiply-adds (error ~1e-16 rad), so that sincos only ever sees |r| <= pi and
// never takes its slow large-argument path.
__device__ __forceinline__ void rope_sincos(int64_t position, double inv_freq, double& s, double& c) {
    const double angle = static_cast<double>(position) * inv_freq;
    const double two_pi_hi = 6.283185307179586232;        // 2*pi rounded to double
    const double two_pi_lo = 2.4492935982947064e-16;      // 2*pi - two_pi_hi
    const double k = rint(angle * 0.15915494309189535);   // 1/(2*pi)
    double r = fma(-k, two_pi_hi, angle);
    r = fma(-k, two_pi_lo, r);
    sincos(r, &s, &c);
}

// Rotate one rotate_half pair at `position` for frequency index i, in double
// (pyfiles/gen_gqa_wrapper_vectors.py:30-34).
__device__ __forceinline__ void rope_pair(double x, double y, int64_t position, double inv_freq,
                                          double& xr, double& yr) {
    double s, c;
    rope_sincos(position, inv_freq, s, c);
    xr = x * c - y * s;
    yr = x * s + y * c;
}


typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef double f64x4_t __attribute__((ext_vector_type(4)));

// BF16 code of a double, rounding through f32 (any nearby BF16 value serves as the
// leading part of a split; the residual is formed exactly in double).
__device__ __forceinline__ uint16_t bf16_of(double d) { return f32_to_bf16_rne(static_cast<float>(d)); }

__device__ __forceinline__ double f64_of_bf16(uint16_t b) { return static_cast<double>(bf16_to_f32(b)); }

__device__ __forceinline__ bf16x8_t pack8(const uint16_t (&h)[8]) {
    union {
        uint16_t u[8];
        bf16x8_t v;
    } t;
#pragma unroll
    for (int j = 0; j < 8; ++j) t.u[j] = h[j];
    return t.v;
}

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4& w) {
    union {
        uint4 u;
        bf16x8_t v;
    } t;
    t.u = w;
    return t.v;
}

// 16-byte load with the nontemporal hint (global_load_dwordx4 ... nt).  Every K/V row
// is read exactly once per step, so the rows should not displace anything in L2 or
// the Infinity Cache; on MI355X the hint raised the stream kernel from 5.5 to 6.1 TB/s
// on the B=64 ragged decode batch.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_stream16(const char* p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

}  // namespace gqa
