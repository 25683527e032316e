// Device math routines of this backend's own, written from the mathematics.
// The header also compiles as plain C++ so the routines can be checked on the
// host against the C library (tests/test_devmath.py builds it with g++).
#pragma once

#ifndef __HIPCC_RTC__ // hipRTC provides the device math and runtime itself
#include <math.h>
#endif

#ifdef __HIPCC__
#define TG_HD __host__ __device__
#else
#define TG_HD
#endif

// log(1 + y) for y in [0, 1] (and NaN), rounded once to f32: the argument of
// softplus's log1pf(expf(-|x|)) is always in that range. Evaluated in f64,
// which issues at the f32 rate on CDNA, instead of the library's compensated
// f32 log1pf:
//   with u = 1 + y, f = u - 1 is y itself when u <= sqrt(2); above, u is
//   halved and ln 2 added, f = (y - 1) / 2 (exact in f64), so u = 1 + f lies
//   in [sqrt(2)/2, sqrt(2)]. With s = f / (2 + f),
//   |s| <= 0.1716, log u = 2 atanh(s) = 2 s (1 + z/3 + z^2/5 + ... + z^9/19)
//   with z = s^2 <= 0.0295; the first omitted term is below 3e-17 of the
//   result, so the f64 value is within a few 1e-16 of log(1 + y) and its f32
//   rounding is the correctly rounded log1pf(y) except within that distance
//   of a rounding boundary.
TG_HD inline float tg_log1p_unit(float y)
{
	double f = (double)y, k = 0.0;
	if (f > 0.41421356237309503) {
		f = (f - 1.0) * 0.5;
		k = 1.0;
	}
	const double s = f / (2.0 + f);
	const double z = s * s;
	double p = 1.0 / 19; // Horner steps as fused multiply-adds, the same on host and device
	p = fma(p, z, 1.0 / 17);
	p = fma(p, z, 1.0 / 15);
	p = fma(p, z, 1.0 / 13);
	p = fma(p, z, 1.0 / 11);
	p = fma(p, z, 1.0 / 9);
	p = fma(p, z, 1.0 / 7);
	p = fma(p, z, 1.0 / 5);
	p = fma(p, z, 1.0 / 3);
	p = fma(p, z, 1.0);
	return (float)(k * 0.6931471805599453 + 2.0 * s * p);
}

#ifdef __HIPCC__
#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>
#endif

// sum of z[0 .. n) in index order, one f32 rounding per add as in a
// sequential loop; z 16-byte aligned (an LDS line). The loop runs in steps of
// 64 NB values, fully unrolled and with no loaded value carried across its
// back edge, so the compiler issues each step's 16-byte loads ahead of its
// adds and only the adds wait on each other (plus one load latency per step).
template <int NB> __device__ __attribute__((always_inline)) inline float tg_ordered_sum(const float *z, int n)
{
	constexpr int S = 64 * NB, B = 32;
	float sum = 0.0f;
	int i = 0;
	for (; i + S <= n; i += S) {
#pragma unroll
		for (int c = 0; c < S / 4; c++) {
			const float4 v = ((const float4 *)(z + i))[c];
			sum += v.x;
			sum += v.y;
			sum += v.z;
			sum += v.w;
		}
	}
	for (; i + B <= n; i += B) {
		float4 v[B / 4];
#pragma unroll
		for (int c = 0; c < B / 4; c++) v[c] = ((const float4 *)(z + i))[c];
#pragma unroll
		for (int c = 0; c < B / 4; c++) {
			sum += v[c].x;
			sum += v[c].y;
			sum += v[c].z;
			sum += v[c].w;
		}
	}
	if (i < n) { // fewer than B left: load them all, then add in order
		float t[B];
#pragma unroll
		for (int k = 0; k < B; k++) t[k] = z[i + k < n ? i + k : n - 1];
#pragma unroll
		for (int k = 0; k < B; k++)
			if (i + k < n) sum += t[k];
	}
	return sum;
}

// The same sum for a single long chain whose loads would otherwise wait on
// each other: values go through two register buffers of 4 V in turn, the
// next buffer's 16-byte loads in flight while the current one's adds run (no
// copy between the buffers, so nothing waits for the loads just issued).
template <int V, bool SQ = false> __device__ __attribute__((always_inline)) inline float tg_ordered_sum_pp(const float *z, int n)
{
	constexpr int W = 4 * V; // values per buffer
	const float4 *z4 = (const float4 *)z;
	const int nb = n / W; // whole buffers
	float sum = 0.0f;
	float4 A[V], B[V];
	auto add = [&](const float4 *v) {
#pragma unroll
		for (int j = 0; j < V; j++) {
			sum += SQ ? v[j].x * v[j].x : v[j].x;
			sum += SQ ? v[j].y * v[j].y : v[j].y;
			sum += SQ ? v[j].z * v[j].z : v[j].z;
			sum += SQ ? v[j].w * v[j].w : v[j].w;
		}
	};
	if (nb > 0)
#pragma unroll
		for (int j = 0; j < V; j++) A[j] = z4[j];
	int b = 0;
	for (; b + 1 < nb; b += 2) {
#pragma unroll
		for (int j = 0; j < V; j++) B[j] = z4[(b + 1) * V + j];
		add(A);
		if (b + 2 < nb)
#pragma unroll
			for (int j = 0; j < V; j++) A[j] = z4[(b + 2) * V + j];
		add(B);
	}
	if (b < nb) add(A); // an odd buffer count ends in A
	const int i = nb * W;
	if (i < n) { // fewer than W left: load them all, then add in order
		float t[W];
#pragma unroll
		for (int k = 0; k < W; k++) t[k] = z[i + k < n ? i + k : n - 1];
#pragma unroll
		for (int k = 0; k < W; k++)
			if (i + k < n) sum += SQ ? t[k] * t[k] : t[k];
	}
	return sum;
}
#endif
