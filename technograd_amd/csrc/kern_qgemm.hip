// Quantized linear layers on the gfx950 int8 matrix cores.
//
// The reference computes o[c] = s[c] * (sum_k (float)code[c][k] * x[k]) with an
// f32 running sum (runtime/tg_rt.h:132-151). Here each activation row is
// written exactly as a 24-bit fixed-point vector q = rint(x * 2^(23-E)) with E
// the row's exponent (max |x| < 2^E), and q is split into three balanced int8
// digits q = d0 + 256 d1 + 65536 d2. v_mfma_i32_16x16x64_i8 sums code * d_l in
// int32 exactly for each digit l; the digit sums are combined in int64, scaled
// by 2^(E-23) in double (exact) and rounded to f32 once, then multiplied by
// the channel scale in f32 like the reference. The only approximation is the
// 24-bit activation grid (error <= 2^-24 max|x| per element), far below the
// reference's own f32 summation error at these K.
//
// Rows with a non-finite or huge entry are flagged by the digit kernel and
// their outputs are recomputed in the epilogue with the reference's exact
// sequential f32 loop, so inf/nan propagate as they do in the reference.
//
// Weight layouts (repacked once at load, channel-major, K padded to 64):
//   int8: w[c][k] = code.
//   int4: 8 bytes per 16 inputs; byte b of group g holds t(16g + b) in its low
//         nibble and t(16g + b + 8) in its high nibble, t = code + 8 in [0, 15]
//         (offset binary), so unpacking is two masks per 4 bytes; the +8 bias
//         is removed with the per-row digit sums: sum t d = sum code d + 8 sum d.
#include "tg_kern.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef int v4i __attribute__((ext_vector_type(4)));

namespace {

constexpr int KB = 64;        // K per MFMA step
constexpr int TILE = 64;      // output tile per workgroup (rows and channels)

inline long round_up(long x, long m) { return (x + m - 1) / m * m; }

struct Scratch {
	int8_t *d[3];   // digit planes [Mp][Kp]
	int *e;         // [Mp] row exponent E
	int *sum;       // [3][Mp] digit sums
	int *special;   // [Mp]
};

Scratch carve(void *base, int Mp, int Kp)
{
	Scratch s;
	char *p = (char *)base;
	for (int l = 0; l < 3; l++) {
		s.d[l] = (int8_t *)p;
		p += (size_t)Mp * Kp;
	}
	s.e = (int *)p;
	p += (size_t)Mp * sizeof(int);
	s.sum = (int *)p;
	p += (size_t)3 * Mp * sizeof(int);
	s.special = (int *)p;
	return s;
}

__device__ inline float xat(const tgk_qgemm_args &a, int m, int k)
{
	long r = m / a.ni, j = m - r * a.ni;
	return a.x[r * a.xr + j * a.xj + (long)k * a.xk];
}

// One workgroup per activation row: exponent, digits, digit sums, special flag.
__global__ __launch_bounds__(256) void digits_k(tgk_qgemm_args a, Scratch s, int K, int Kp, int M)
{
	__shared__ float red[256];
	__shared__ int ired[3][256];
	__shared__ int bad;
	int m = blockIdx.x, t = threadIdx.x;
	if (t == 0) bad = 0;
	__syncthreads();
	float mx = 0.0f;
	if (m < M)
		for (int k = t; k < K; k += 256) {
			float v = xat(a, m, k);
			if (!isfinite(v)) bad = 1;
			mx = fmaxf(mx, fabsf(v));
		}
	red[t] = mx;
	__syncthreads();
	for (int w = 128; w > 0; w >>= 1) {
		if (t < w) red[t] = fmaxf(red[t], red[t + w]);
		__syncthreads();
	}
	float amax = red[0];
	int special = bad || amax > 0x1p100f;
	int E = 0;
	double sc = 1.0;
	if (!special && amax > 0.0f) {
		frexpf(amax, &E); // amax = f 2^E, f in [0.5, 1)
		sc = ldexp(1.0, 23 - E);
		if (rint((double)amax * sc) > 8355328.0) { // keep the top digit within int8
			E += 1;
			sc = ldexp(1.0, 23 - E);
		}
	}
	int s0 = 0, s1 = 0, s2 = 0;
	for (int k = t; k < Kp; k += 256) {
		int q = 0;
		if (m < M && k < K && !special) q = (int)rint((double)xat(a, m, k) * sc);
		int d0 = (int)(int8_t)(q & 255);
		int q1 = (q - d0) >> 8;
		int d1 = (int)(int8_t)(q1 & 255);
		int d2 = (q1 - d1) >> 8;
		long off = (long)m * Kp + k;
		s.d[0][off] = (int8_t)d0;
		s.d[1][off] = (int8_t)d1;
		s.d[2][off] = (int8_t)d2;
		s0 += d0;
		s1 += d1;
		s2 += d2;
	}
	ired[0][t] = s0;
	ired[1][t] = s1;
	ired[2][t] = s2;
	__syncthreads();
	for (int w = 128; w > 0; w >>= 1) {
		if (t < w)
			for (int l = 0; l < 3; l++) ired[l][t] += ired[l][t + w];
		__syncthreads();
	}
	if (t == 0) {
		s.e[m] = E;
		s.special[m] = special;
		for (int l = 0; l < 3; l++) s.sum[(long)l * gridDim.x + m] = ired[l][0];
	}
}

__device__ inline int code_orig(const tgk_qweight &w, int c, int k)
{
	long i = w.axis == 0 ? (long)c * w.K + k : (long)k * w.C + c;
	if (w.bits == 8) return (signed char)w.orig[i];
	int b = (signed char)w.orig[i >> 1];
	return (i & 1) ? (b >> 4) : (int)(signed char)(unsigned char)((unsigned)b << 4) >> 4;
}

template <int BITS>
__device__ inline v4i load_w(const uint8_t *w, int Kp, int c, int k)
{
	if (BITS == 8) return *(const v4i *)(w + (long)c * Kp + k);
	const unsigned *p = (const unsigned *)(w + (long)c * (Kp / 2) + k / 2);
	unsigned w0 = p[0], w1 = p[1];
	v4i r;
	r.x = (int)(w0 & 0x0f0f0f0fu);
	r.y = (int)(w1 & 0x0f0f0f0fu);
	r.z = (int)((w0 >> 4) & 0x0f0f0f0fu);
	r.w = (int)((w1 >> 4) & 0x0f0f0f0fu);
	return r;
}

// 256 threads = 4 waves; the workgroup computes a 64 x 64 output tile, each
// wave a 32 x 32 quarter as 2 x 2 MFMA blocks of 16 x 16, three digit planes.
template <int BITS>
__global__ __launch_bounds__(256) void qgemm_k(tgk_qgemm_args a, tgk_qweight w, Scratch s, int Mp)
{
	const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
	const int m0 = blockIdx.y * TILE + (wave >> 1) * 32, c0 = blockIdx.x * TILE + (wave & 1) * 32;
	const int Kp = w.Kp, row16 = lane & 15, kq = (lane >> 4) * 16;
	v4i acc[3][2][2];
	for (int l = 0; l < 3; l++)
		for (int i = 0; i < 2; i++)
			for (int j = 0; j < 2; j++) acc[l][i][j] = v4i{ 0, 0, 0, 0 };
	for (int k0 = 0; k0 < Kp; k0 += KB) {
		v4i bw[2], ad[3][2];
		for (int j = 0; j < 2; j++) bw[j] = load_w<BITS>(w.w, Kp, c0 + j * 16 + row16, k0 + kq);
		for (int l = 0; l < 3; l++)
			for (int i = 0; i < 2; i++) ad[l][i] = *(const v4i *)(s.d[l] + (long)(m0 + i * 16 + row16) * Kp + k0 + kq);
		for (int l = 0; l < 3; l++)
			for (int i = 0; i < 2; i++)
				for (int j = 0; j < 2; j++) acc[l][i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ad[l][i], bw[j], acc[l][i][j], 0, 0, 0);
	}
	const long corr = BITS == 4 ? 8 : 0;
	for (int i = 0; i < 2; i++)
		for (int j = 0; j < 2; j++)
			for (int v = 0; v < 4; v++) {
				int m = m0 + i * 16 + (lane >> 4) * 4 + v, c = c0 + j * 16 + row16;
				if (m >= a.M || c >= w.C) continue;
				float acc32;
				if (s.special[m]) {
					float t = 0.0f;
					for (int k = 0; k < w.K; k++) t += (float)code_orig(w, c, k) * xat(a, m, k);
					acc32 = t;
				} else {
					long t0 = (long)acc[0][i][j][v] - corr * s.sum[m];
					long t1 = (long)acc[1][i][j][v] - corr * s.sum[(long)Mp + m];
					long t2 = (long)acc[2][i][j][v] - corr * s.sum[2L * Mp + m];
					long tot = t0 + t1 * 256 + t2 * 65536;
					acc32 = (float)ldexp((double)tot, s.e[m] - 23);
				}
				long r = m / a.ni, jj = m - r * a.ni;
				a.o[r * a.orr + (long)c * a.oc + jj * a.oj] = w.scale[c] * acc32;
			}
}

} // namespace

int tgk_qweight_pack(tgk_qweight *w, const uint8_t *codes, const float *scale, int bits, int axis, int C, int K, hipStream_t st)
{
	memset(w, 0, sizeof *w);
	w->C = C;
	w->K = K;
	w->bits = bits;
	w->axis = axis;
	w->Kp = (int)round_up(K, KB);
	w->Cp = (int)round_up(C, TILE);
	size_t rowb = bits == 8 ? (size_t)w->Kp : (size_t)w->Kp / 2;
	size_t nb = (size_t)w->Cp * rowb, ob = bits == 8 ? (size_t)C * K : ((size_t)C * K + 1) / 2;
	uint8_t *h = (uint8_t *)calloc(nb, 1);
	float *hs = (float *)calloc((size_t)w->Cp, sizeof(float));
	if (!h || !hs) {
		free(h);
		free(hs);
		return -1;
	}
	for (int c = 0; c < C; c++) {
		uint8_t *row = h + (size_t)c * rowb;
		if (bits == 4)
			for (size_t b = 0; b < rowb; b++) row[b] = 0x88; /* padding codes 0 */
		for (int k = 0; k < K; k++) {
			long i = axis == 0 ? (long)c * K + k : (long)k * C + c;
			int code;
			if (bits == 8) code = (signed char)codes[i];
			else {
				int b = (signed char)codes[i >> 1];
				code = (i & 1) ? (b >> 4) : (int)(signed char)(unsigned char)((unsigned)b << 4) >> 4;
			}
			if (bits == 8) {
				row[k] = (uint8_t)(int8_t)code;
			} else {
				int g = k / 16, r = k % 16, byte = g * 8 + (r & 7);
				unsigned t = (unsigned)(code + 8);
				row[byte] = r < 8 ? (uint8_t)((row[byte] & 0xf0) | t) : (uint8_t)((row[byte] & 0x0f) | (t << 4));
			}
		}
		hs[c] = scale[c];
	}
	int rc = 0;
	if (hipMalloc(&w->w, nb) != hipSuccess || hipMalloc(&w->scale, (size_t)w->Cp * sizeof(float)) != hipSuccess ||
	    hipMalloc(&w->orig, ob) != hipSuccess)
		rc = -1;
	if (!rc && (hipMemcpyAsync(w->w, h, nb, hipMemcpyHostToDevice, st) != hipSuccess ||
		    hipMemcpyAsync(w->scale, hs, (size_t)w->Cp * sizeof(float), hipMemcpyHostToDevice, st) != hipSuccess ||
		    hipMemcpyAsync(w->orig, codes, ob, hipMemcpyHostToDevice, st) != hipSuccess || hipStreamSynchronize(st) != hipSuccess))
		rc = -1;
	free(h);
	free(hs);
	return rc;
}

void tgk_qweight_free(tgk_qweight *w)
{
	if (w->w) hipFree(w->w);
	if (w->scale) hipFree(w->scale);
	if (w->orig) hipFree(w->orig);
	memset(w, 0, sizeof *w);
}

size_t tgk_qgemm_scratch(int M, int Kp)
{
	long Mp = round_up(M, TILE);
	return (size_t)Mp * Kp * 3 + (size_t)Mp * sizeof(int) * 5 + 256;
}

void tgk_qgemm_digits(hipStream_t st, const tgk_qgemm_args *a, void *scratch)
{
	const tgk_qweight *w = a->w;
	if (!w || !w->w || !a->x || !scratch || a->M <= 0 || a->ni <= 0) return; /* nothing valid to launch */
	int Mp = (int)round_up(a->M, TILE);
	digits_k<<<Mp, 256, 0, st>>>(*a, carve(scratch, Mp, w->Kp), w->K, w->Kp, a->M);
}

void tgk_qgemm_mfma(hipStream_t st, const tgk_qgemm_args *a, void *scratch)
{
	const tgk_qweight *w = a->w;
	if (!w || !w->w || !w->scale || !a->x || !a->o || !scratch || a->M <= 0 || a->ni <= 0) return;
	int Mp = (int)round_up(a->M, TILE);
	Scratch s = carve(scratch, Mp, w->Kp);
	dim3 grid(w->Cp / TILE, Mp / TILE);
	if (w->bits == 8) qgemm_k<8><<<grid, 256, 0, st>>>(*a, *w, s, Mp);
	else qgemm_k<4><<<grid, 256, 0, st>>>(*a, *w, s, Mp);
}

void tgk_qgemm(hipStream_t st, const tgk_qgemm_args *a, void *scratch)
{
	tgk_qgemm_digits(st, a, scratch);
	tgk_qgemm_mfma(st, a, scratch);
}
