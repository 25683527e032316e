// Per-lane numerics of the row programs: the Q16.16 primitives of the
// fixed-point runtime (runtime/tg_rtq.h:30-145 restated), the f32 element
// functions of the reference's kernels (runtime/tg_rt.h:40-64) and the qcode
// nibble rule. Shared by the row-program interpreter (kern_rowprog.hip) and by
// the row programs compiled for one model at load time (tg_rpgen.cpp), which
// hand this file and tg_devmath.h to hipRTC as they are, so both executors
// run the same element code.
//
// Constants are derived from their definitions at compile time: ln 2, pi,
// pi/2, 2 pi, 0.044715 and 0.7978845608 rounded to Q16, 1e-6 in Q32, the exp
// series round(2^30 / j!) in Q30, and exp's cut-offs (above ln 32768 in Q16
// the result saturates, below -12 it is 0).
#pragma once

#include "tg_devmath.h"

namespace tgrd {

constexpr int ONE = 65536;
constexpr int MAXV = 2147483647;
constexpr int MINV = -2147483647 - 1;

// round(v * 2^16) for v > 0
constexpr long q16(double v) { return (long)(v * 65536.0 + 0.5); }
// round(2^30 / j!) = floor((2^31 + j!) / (2 j!))
constexpr long expc(int j)
{
	long f = 1;
	for (int i = 2; i <= j; i++) f *= i;
	return ((1L << 31) + f) / (2 * f);
}

constexpr long LN2 = q16(0.6931471805599453), PIQ = q16(3.141592653589793), HPIQ = q16(1.5707963267948966),
	       TPIQ = q16(6.283185307179586);
constexpr long GELU_A = q16(0.044715), GELU_B = q16(0.7978845608);
constexpr unsigned long EPS_Q32 = (unsigned long)(1e-6 * 4294967296.0 + 0.5);
constexpr int EXP_HI = (int)q16(15 * 0.6931471805599453), EXP_LO = -12 * ONE;

// Two device operations with host stand-ins for the host builds of this
// header (tests): an approximate f32 reciprocal and the low 32 bits of a
// 24 x 24-bit product. fdivq_unit gives the same result with either.
#ifdef __HIP_DEVICE_COMPILE__
#define TGRD_RCP(x) __builtin_amdgcn_rcpf(x)
#define TGRD_MUL24(a, b) __umul24((a) & 0xffffffu, (b) & 0xffffffu) // operands below 2^24: the masks fold away
#else
#define TGRD_RCP(x) (1.0f / (x))
#define TGRD_MUL24(a, b) ((a) * (b))
#endif

__device__ inline int sat(long v) { return v > MAXV ? MAXV : v < MINV ? MINV : (int)v; }
// saturating int32 add and subtract: sat((long)x +- y), one clamped instruction
__device__ inline int addq(int x, int y) { return __builtin_elementwise_add_sat(x, y); }
__device__ inline int subq(int x, int y) { return __builtin_elementwise_sub_sat(x, y); }
__device__ inline int fmulq(int a, int b) { return sat(((long)a * b + 32768) >> 16); }
__device__ inline int fdivq(int a, int b)
{
	if (b == 0) return a > 0 ? MAXV : a < 0 ? MINV : 0;
	long n = (long)a * 65536, h = b > 0 ? b / 2 : -(b / 2);
	return sat(((n >= 0) == (b > 0) ? n + h : n - h) / b);
}
__device__ inline int absq(int a) { return a < 0 ? subq(0, a) : a; } // |MINV| saturates to MAXV

// the high 32 bits of a 32 x 32-bit product (one instruction)
__device__ inline unsigned mulhi(unsigned a, unsigned b) { return (unsigned)(((unsigned long)a * b) >> 32); }

// exp's degree-8 Horner polynomial in Q30 at f = r4 / 2^32 in [0, ln 2), r4 =
// 4 r for the runtime's reduced argument r = f 2^30 < 2^30. Every Horner value
// lies below 2^31 (a truncated series of e^f < 2), so each step's
// (p * r) >> 30 of the runtime's int64 arithmetic equals mulhi(p, 4 r).
__device__ inline unsigned exp_poly(unsigned r4)
{
	unsigned p = (unsigned)expc(8);
	p = (unsigned)expc(7) + mulhi(p, r4);
	p = (unsigned)expc(6) + mulhi(p, r4);
	p = (unsigned)expc(5) + mulhi(p, r4);
	p = (unsigned)expc(4) + mulhi(p, r4);
	p = (unsigned)expc(3) + mulhi(p, r4);
	p = (unsigned)expc(2) + mulhi(p, r4);
	p = (unsigned)expc(1) + mulhi(p, r4);
	return (unsigned)expc(0) + mulhi(p, r4);
}

__device__ inline int expq(int x)
{
	if (x > EXP_HI) return MAXV;
	if (x < EXP_LO) return 0;
	long k = x >= 0 ? x / LN2 : -((-(long)x + LN2 - 1) / LN2);
	const long p = exp_poly((unsigned)(((long)x - k * LN2) * 65536));
	int sh = (int)k - 14;
	long v = sh >= 0 ? p * (1L << sh) : (p + (1L << (-sh - 1))) >> -sh;
	return sat(v);
}

// expq for x <= 0 in 32-bit arithmetic. With m = -x in [0, 12 ONE] and
// k = -floor(x / ln 2) = ceil(m / ln 2) in [0, 18], the reduced argument
// k ln2 - m lies in [0, ln2), the polynomial stays below 2^31, the rounding
// bias 2^(13 + k) <= 2^31 and the sum below 2^32; at k = 18 the shift is 32
// and the result 0. Equal to expq on [-12 ONE, 0].
__device__ inline int expq_neg(int x)
{
	if (x < EXP_LO) return 0;
	const unsigned m = (unsigned)-x, k = (m + (unsigned)LN2 - 1) / (unsigned)LN2;
	const unsigned p = exp_poly((k * (unsigned)LN2 - m) * 65536u);
	const unsigned sh = 14 + k;
	return sh >= 32 ? 0 : (int)((p + (1u << (sh - 1))) >> sh);
}

__device__ inline int logq(int x)
{
	if (x <= 0) return MINV;
	int e = 0;
	unsigned m = (unsigned)x;
	while (m >= 131072u) {
		m >>= 1;
		e++;
	}
	while (m < 65536u) {
		m <<= 1;
		e--;
	}
	long s = ((long)(m - 65536) << 30) / (long)(m + 65536), s2 = (s * s) >> 30, t = s, acc = 0;
	for (int k = 1; k <= 13; k += 2) {
		acc += t / k;
		t = (t * s2) >> 30;
	}
	return sat(((2 * acc) >> 14) + (long)e * LN2);
}

__device__ inline unsigned long isqrt64(unsigned long v)
{
	unsigned long r = 0, bit = 1UL << 62;
	while (bit > v) bit >>= 2;
	while (bit) {
		if (v >= r + bit) {
			v -= r + bit;
			r = (r >> 1) + bit;
		} else {
			r >>= 1;
		}
		bit >>= 2;
	}
	return r;
}

__device__ inline int sinq(int x)
{
	long r = (long)x % TPIQ;
	if (r > PIQ) r -= TPIQ;
	if (r < -PIQ) r += TPIQ;
	if (r > HPIQ) r = PIQ - r;
	if (r < -HPIQ) r = -PIQ - r;
	long z = r * 16384, z2 = (z * z) >> 30, t = z, acc = 0;
	for (int k = 1; k <= 13; k += 2) {
		acc += t;
		t = -((t * z2) >> 30) / ((k + 1) * (k + 2));
	}
	return sat((acc + 8192) >> 14);
}

// floor(n / d) for 0 <= n < 2^53, 0 < d < 2^35 and n / d < 2^17: n and d are
// exact in f64, the correctly rounded quotient is within 2^-36 of n / d, and
// a non-integer n / d is at least 1/d > 2^-35 from the next integer, so the
// f64 quotient truncates to the integer one.
__device__ inline long divsmall(long n, long d) { return (long)((double)n / (double)d); }

// fdivq(a, b) for 0 <= a <= ONE <= b <= 2 ONE (quotients of exp values):
// floor((a 2^16 + floor(b / 2)) / b) <= 2^16 + 1, never saturated. The f32
// estimate has a relative error below 2^-21 (the rounded numerator, an
// approximate reciprocal within 1 ulp, the product), so it is within 2^-5 of
// the quotient and truncates to it or a neighbour; the remainder, in
// (-b, 2b) and hence exact in wrapping 32-bit arithmetic, corrects it.
__device__ inline int fdivq_unit(int a, int b)
{
	const unsigned h = (unsigned)b >> 1;
	const unsigned q = (unsigned)(((float)a * 65536.0f + (float)h) * TGRD_RCP((float)b));
	const int r = (int)((unsigned)a * 65536u + h - TGRD_MUL24(q, (unsigned)b));
	return (int)q + (r >= b) - (r < 0);
}

__device__ inline int tanhq(int x)
{
	int t = absq(x);
	if (t > 9 * ONE) return x < 0 ? -ONE : ONE;
	int e = expq_neg(-2 * t); // in [0, ONE]
	int y = fdivq_unit(ONE - e, ONE + e);
	return x < 0 ? -y : y;
}

__device__ inline int sigmoidq(int x)
{
	int e = expq_neg(-absq(x)); // in [0, ONE]
	return x >= 0 ? fdivq_unit(ONE, ONE + e) : fdivq_unit(e, ONE + e);
}

__device__ inline int geluq(int x)
{
	long v = x, x3 = (((v * v) >> 16) * v) >> 16;
	long u = ((v + ((x3 * GELU_A) >> 16)) * GELU_B) >> 16;
	int t = tanhq(sat(u));
	return sat((v * ((long)ONE + t)) >> 17);
}

__device__ inline int negq(int x) { return subq(0, x); }
__device__ inline int reluq(int x) { return x > 0 ? x : 0; }
__device__ inline int sqrtq(int x) { return x > 0 ? (int)isqrt64((unsigned long)x << 16) : 0; }
__device__ inline int siluq(int x) { return fmulq(x, sigmoidq(x)); }
__device__ inline int softplusq(int x) { return sat((long)(x > 0 ? x : 0) + logq(ONE + expq_neg(-absq(x)))); }
__device__ inline int cosq(int x) { return sinq(sat((long)x + HPIQ)); }
__device__ inline int floorq(int x) { return (int)((unsigned)x & 0xffff0000u); }
__device__ inline int stepq(int x) { return x > 0 ? ONE : 0; }
__device__ inline int maxq(int x, int y) { return x > y ? x : y; }
__device__ inline int minq(int x, int y) { return x < y ? x : y; }

// rmsnorm's root of one line from its sum of squares in Q32:
// isqrt64(ss / cols + 1e-6 in Q32), never 0 (runtime/tg_rtq.h:214-225)
__device__ inline int rmsq(unsigned long ss, int cols)
{
	const int rms = (int)isqrt64(ss / (unsigned long)cols + EPS_Q32);
	return rms > 0 ? rms : 1;
}

// softmax's normalisation of one exp value 0 <= y <= ONE by the line's sum
// s >= ONE of such values: the quotient is at most 2^16 + 1, so divsmall
// applies while s < 2^35 (lines of fewer than 2^19 elements)
__device__ inline int softq(long y, long s)
{
	const long n = y * 65536 + s / 2;
	return (int)(s < (1L << 35) ? divsmall(n, s) : n / s);
}

// the Q7.24 channel scale applied to an int64 code sum: sat((acc * s + 2^23) >> 24)
__device__ inline int qscaleq(long acc, int s)
{
	return sat(((long)((unsigned long)acc * (unsigned long)(long)s) + (1L << 23)) >> 24);
}

// code i of a quantized param: int8, or int4 packed two per byte, low nibble first
__device__ inline int qcode(const unsigned char *q, int bits, long i)
{
	if (bits == 8) return (signed char)q[i];
	int b = (signed char)q[i >> 1];
	return (i & 1) ? (b >> 4) : (int)(signed char)(unsigned char)((unsigned)b << 4) >> 4;
}

// f32 element functions as the reference's kernels write them
// (runtime/tg_rt.h:40-64); libm calls are the device library's
__device__ inline float negf_(float x) { return -x; }
__device__ inline float reluf_(float x) { return x > 0.0f ? x : 0.0f; }
__device__ inline float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ inline float geluf_(float x) { return 0.5f * x * (1.0f + tanhf(0.7978845608f * (x + 0.044715f * x * x * x))); }
__device__ inline float siluf_(float x) { return x / (1.0f + expf(-x)); }
__device__ inline float softplusf_(float x) { return (x > 0.0f ? x : 0.0f) + tg_log1p_unit(expf(-fabsf(x))); }
__device__ inline float stepf_(float x) { return x > 0.0f ? 1.0f : 0.0f; }
__device__ inline float maxf_(float x, float y) { return x > y ? x : y; }
__device__ inline float minf_(float x, float y) { return x < y ? x : y; }

} // namespace tgrd
