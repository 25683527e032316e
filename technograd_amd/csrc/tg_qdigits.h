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

// digits of 16 consecutive inputs (inputs k0 .. k0 + 15 of the row at blk)
// into their three 16-byte chunks; zero digits when `zero`; returns the sum of q
__device__ inline long long tgq_put16(int8_t *blk, int k0, const float *v, int E, bool zero)
{
	unsigned w0[4] = {0, 0, 0, 0}, w1[4] = {0, 0, 0, 0}, w2[4] = {0, 0, 0, 0};
	int qs = 0; // |sum of 16 q| < 2^27
	if (!zero) {
		for (int i = 0; i < 16; i++) {
			const int q = (int)rintf(ldexpf(v[i], 23 - E)); // exact: |q| < 2^23
			qs += q;
			int d0, d1, d2;
			tgq_split3(q, d0, d1, d2);
			const int sh = (i & 3) * 8;
			w0[i >> 2] |= (unsigned)(d0 & 255) << sh;
			w1[i >> 2] |= (unsigned)(d1 & 255) << sh;
			w2[i >> 2] |= (unsigned)(d2 & 255) << sh;
		}
	}
	int8_t *p = blk + (k0 >> 5) * 3072 + ((k0 >> 4) & 1) * 512;
	*(tgq_v4i *)p = tgq_v4i{(int)w0[0], (int)w0[1], (int)w0[2], (int)w0[3]};
	*(tgq_v4i *)(p + 1024) = tgq_v4i{(int)w1[0], (int)w1[1], (int)w1[2], (int)w1[3]};
	*(tgq_v4i *)(p + 2048) = tgq_v4i{(int)w2[0], (int)w2[1], (int)w2[2], (int)w2[3]};
	return qs;
}
