// Activation digits of the exact int8 matrix-core GEMM (kern_qgemm.hip), as
// device functions shared by the GEMM's digit kernels and the fused decode
// kernels, so every producer writes the same bytes.
//
// A row x of K inputs is written as q_k = rint(x_k 2^(23-E)), E the row's
// exponent (max |x| = f 2^E, f in [0.5, 1), raised by one when the top digit
// would leave int8), and each q as three balanced base-256 int8 digits. Rows
// with a non-finite entry or max |x| above 2^100 are "special": their digits
// are zero and the GEMM's epilogue runs the reference's sequential loop.
//
// Peaked rows are special too. The grid step 2^(E-23) is set by the largest
// entry; when a few entries stand far above all the others (an outlier
// channel), the others lose precision on that grid, and the reference's
// sequential sum, which never sees the outlier on a channel whose code is 0,
// would be the more accurate. The band of a row is |x| >= max|x| / 4. A row
// is peaked when some nonzero entry lies below its band and at most
// tgq_peak_max(K) entries lie in it (8, or max(1, K / 4) for K < 32): then
// max|x| is at most 4 times the row's 9th largest |x| (its largest for
// short rows), so the grid step stays within a small factor of what the
// bulk of the row would set. Gaussian-like rows of 64 or more entries are
// never peaked (the band holds about a third of them), rows whose entries
// are a few values and zeros (one-hot, {0, 1}) neither; a single entry 14
// or more standard deviations out is. Every quantity is a count, so the
// decision does not depend on the order of any sum. Peaked rows are found
// after their digits are written (the counts come with the sum of q); their
// digits are then unused.
//
// Layout (the MFMA fragment order of v_mfma_i32_32x32x32_i8):
//   digits [row / 32][k / 32][digit 0..2][lane 0..63][16 bytes],
//   lane = row % 32 + 32 ((k % 32) / 16).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef int tgq_v4i __attribute__((ext_vector_type(4)));

// balanced base-256 digits of |q| < 2^23: q = d0 + 256 d1 + 65536 d2, d_l in [-128, 127]
__device__ inline void tgq_split3(int q, int &d0, int &d1, int &d2)
{
	d0 = (int)(int8_t)(q & 255);
	const int q1 = (q - d0) >> 8;
	d1 = (int)(int8_t)(q1 & 255);
	d2 = (q1 - d1) >> 8;
}

// a row is special when an entry is not finite (bad) or max |x| exceeds 2^100
__device__ inline int tgq_special(int bad, float amax) { return bad || amax > 0x1p100f; }

// the peak test (see above): the band's floor, the per-16 tally (entries in
// the band + 2^32 nonzero entries below it), and the decision from a row's
// whole tally
constexpr int TGQ_BAND_SHIFT = 2, TGQ_PEAK_N = 8;
__device__ inline float tgq_band(float amax) { return ldexpf(amax, -TGQ_BAND_SHIFT); }
__device__ inline int tgq_peak_max(int K) { return K >= 4 * TGQ_PEAK_N ? TGQ_PEAK_N : K >= 8 ? K >> 2 : 1; }
__device__ inline long long tgq_tally16(const float *v, float band)
{
	int in = 0, below = 0;
	for (int i = 0; i < 16; i++) {
		const float a = fabsf(v[i]);
		in += a >= band && a != 0.0f;
		below += a < band && a != 0.0f;
	}
	return (long long)in + ((long long)below << 32);
}
__device__ inline int tgq_peaked(long long tally, int K) { return (tally >> 32) > 0 && (tally & 0xffffffffll) <= tgq_peak_max(K); }

// the row exponent E from max |x| (0 for special or all-zero rows)
__device__ inline int tgq_exponent(float amax, int special)
{
	int E = 0;
	if (!special && amax > 0.0f) {
		frexpf(amax, &E); // amax = f 2^E, f in [0.5, 1)
		if (rintf(ldexpf(amax, 23 - E)) > 8355328.0f) E += 1; // keep the top digit within int8
	}
	return E;
}

// row m's first fragment byte in a digit area of Kp inputs per row
__device__ inline int8_t *tgq_row_base(int8_t *dig, int m, int Kp) { return dig + (long)(m >> 5) * (Kp / 32) * 3072 + (m & 31) * 16; }

// Row scan: the running max of |x| over a lane's inputs, kept as the bit
// pattern of |x| (unsigned order is the order of magnitudes, and every NaN
// pattern lies above +inf's 0x7f800000): two inputs per max3, no compare.
__device__ inline void tgq_scan16(const float *v, unsigned &mb)
{
	for (int i = 0; i < 16; i += 2) {
		const unsigned a = __float_as_uint(v[i]) & 0x7fffffffu, b = __float_as_uint(v[i + 1]) & 0x7fffffffu;
		mb = max(mb, max(a, b));
	}
}

// four inputs' u = q + 0x808080 -> their digit bytes in the three plane words
// (byte i of plane l's word: d_l of input i; the layout tgq_put16 writes)
__device__ inline void tgq_pack4(const unsigned *u, unsigned &w0, unsigned &w1, unsigned &w2)
{
	const unsigned t01 = __builtin_amdgcn_perm(u[1], u[0], 0x05010400u); // u0.b0 u1.b0 u0.b1 u1.b1
	const unsigned t23 = __builtin_amdgcn_perm(u[3], u[2], 0x05010400u); // u2.b0 u3.b0 u2.b1 u3.b1
	const unsigned s01 = __builtin_amdgcn_perm(u[1], u[0], 0x0c0c0602u); // u0.b2 u1.b2 0 0
	const unsigned s23 = __builtin_amdgcn_perm(u[3], u[2], 0x06020c0cu); // 0 0 u2.b2 u3.b2
	w0 = __builtin_amdgcn_perm(t23, t01, 0x05040100u) ^ 0x80808080u;
	w1 = __builtin_amdgcn_perm(t23, t01, 0x07060302u) ^ 0x80808080u;
	w2 = (s01 | s23) ^ 0x80808080u;
}

// a lane's max |x| and NaN flag from its scan (a NaN lane's max is not used:
// the flag makes the row special). An infinite input is not flagged here: it
// makes max |x| infinite, which tgq_special treats as special all the same.
__device__ inline void tgq_scan_end(unsigned mb, float &mx, int &nan)
{
	nan = mb > 0x7f800000u;
	mx = nan ? 0.0f : __uint_as_float(mb);
}

// the digit words of 16 consecutive inputs: w_l[g] holds plane l's digits of
// inputs 4 g .. 4 g + 3 (byte i: input 4 g + i); returns the sum of q and
// adds the inputs' peak tally (band = tgq_band(max |x|)) to `tally`.
// With u = q + 0x808080 (|q| <= 8355328, so 0 <= u < 2^24), byte l of u is
// d_l + 128: the balanced digits are u's bytes with the top bit flipped. The
// bytes of four inputs are gathered into each plane's 32-bit word with byte
// permutes (v_perm_b32 selects bytes of a register pair: 0-3 the second
// operand's, 4-7 the first's, 12 a zero byte).
__device__ inline long long tgq_digits16(const float *v, int E, float band, unsigned (&w0)[4], unsigned (&w1)[4], unsigned (&w2)[4],
					 long long &tally)
{
	tally += tgq_tally16(v, band);
	int qs = 0; // |sum of 16 q| < 2^27
	for (int g = 0; g < 4; g++) {
		unsigned u[4];
		for (int i = 0; i < 4; i++) {
			const int q = (int)rintf(ldexpf(v[4 * g + i], 23 - E)); // exact: |q| < 2^23
			qs += q;
			u[i] = (unsigned)(q + 0x808080);
		}
		tgq_pack4(u, w0[g], w1[g], w2[g]);
	}
	return qs;
}

// digits of 16 consecutive inputs (inputs k0 .. k0 + 15 of the row at blk)
// into their three 16-byte chunks of the fragment layout; zero digits when
// `zero`; returns the sum of q and adds the inputs' peak tally to `tally`
// (nothing for a `zero` group).
__device__ inline long long tgq_put16(int8_t *blk, int k0, const float *v, int E, bool zero, float band, long long &tally)
{
	int8_t *p = blk + (k0 >> 5) * 3072 + ((k0 >> 4) & 1) * 512;
	if (__builtin_expect(zero, 0)) {
		*(tgq_v4i *)p = tgq_v4i{0, 0, 0, 0};
		*(tgq_v4i *)(p + 1024) = tgq_v4i{0, 0, 0, 0};
		*(tgq_v4i *)(p + 2048) = tgq_v4i{0, 0, 0, 0};
		return 0;
	}
	unsigned w0[4], w1[4], w2[4];
	const long long qs = tgq_digits16(v, E, band, w0, w1, w2, tally);
	*(tgq_v4i *)p = tgq_v4i{(int)w0[0], (int)w0[1], (int)w0[2], (int)w0[3]};
	*(tgq_v4i *)(p + 1024) = tgq_v4i{(int)w1[0], (int)w1[1], (int)w1[2], (int)w1[3]};
	*(tgq_v4i *)(p + 2048) = tgq_v4i{(int)w2[0], (int)w2[1], (int)w2[2], (int)w2[3]};
	return qs;
}
