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
// Operand layouts in global memory are the MFMA fragment order of
// v_mfma_i32_32x32x32_i8 (lane l holds row or channel l % 32 and inputs
// 16 (l / 32) .. +15 of a 32-input block), so the K loop copies contiguous
// 1 KiB chunks straight into LDS (global_load_lds_dwordx4) and every fragment
// read is one contiguous 16- or 8-byte lane read:
//   digits   [row / 32][k / 32][digit 0..2][lane 0..63][16 bytes]
//   int8 w   [channel / 32][k / 32][lane][16 codes]
//   int4 w   [channel / 32][k / 32][lane][8 bytes]: byte b holds t(b) in its
//            low nibble and t(b + 8) in its high nibble of the lane's 16
//            inputs, t = code + 8 in [0, 15] (offset binary), so unpacking is
//            two masks per 4 bytes; the +8 bias is removed with the per-row
//            digit sums: sum t d = sum code d + 8 sum d.
// Weights are repacked once at load (channels padded to 128, K to 64).
#include "tg_kern.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef int v4i __attribute__((ext_vector_type(4)));

namespace {

constexpr int KB = 64;        // inputs per K step of the MFMA kernel
constexpr int BM = 128;       // rows (activations) per workgroup tile
constexpr int BN = 128;       // channels per workgroup tile (weights are padded to it)

inline long round_up(long x, long m) { return (x + m - 1) / m * m; }

typedef int v16i __attribute__((ext_vector_type(16)));
#define LDSP(p) ((__attribute__((address_space(3))) void *)(p))

struct Scratch {
	int8_t *dig;    // digits in fragment order (see above)
	int *e;         // [Mp] row exponent E
	int *sum;       // [3][Mp] digit sums
	int *special;   // [Mp]
};

Scratch carve(void *base, int Mp, int Kp)
{
	Scratch s;
	char *p = (char *)base;
	s.dig = (int8_t *)p;
	p += (size_t)Mp * Kp * 3;
	s.e = (int *)p;
	p += (size_t)Mp * sizeof(int);
	s.sum = (int *)p;
	p += (size_t)3 * Mp * sizeof(int);
	s.special = (int *)p;
	return s;
}

// element k of activation row m
__device__ inline const float *xrow(const tgk_qgemm_args &a, int m)
{
	int r = m / a.ni, j = m - r * a.ni;
	return a.x + (long)r * a.xr + (long)j * a.xj;
}

// One workgroup per activation row: exponent, digits, digit sums, special flag.
__global__ __launch_bounds__(256) void digits_k(tgk_qgemm_args a, Scratch s, int K, int Kp, int M)
{
	__shared__ float red[256];
	__shared__ int ired[3][256];
	__shared__ int bad;
	const int m = blockIdx.x, t = threadIdx.x;
	const float *x = m < M ? xrow(a, m) : a.x;
	const long xk = a.xk;
	if (t == 0) bad = 0;
	__syncthreads();
	float mx = 0.0f;
	if (m < M)
		for (int k = t; k < K; k += 256) {
			float v = x[k * xk];
			if (!isfinite(v)) bad = 1;
			mx = fmaxf(mx, fabsf(v));
		}
	red[t] = mx;
	__syncthreads();
	for (int w = 128; w > 0; w >>= 1) {
		if (t < w) red[t] = fmaxf(red[t], red[t + w]);
		__syncthreads();
	}
	const float amax = red[0];
	const int special = bad || amax > 0x1p100f;
	int E = 0;
	if (!special && amax > 0.0f) {
		frexpf(amax, &E); // amax = f 2^E, f in [0.5, 1)
		if (rintf(ldexpf(amax, 23 - E)) > 8355328.0f) E += 1; // keep the top digit within int8
	}
	int s0 = 0, s1 = 0, s2 = 0;
	const int kblocks = Kp / 32, r = m & 31;
	int8_t *blk = s.dig + (long)(m >> 5) * kblocks * 3072;
	for (int k = t; k < Kp; k += 256) {
		int q = 0;
		if (m < M && k < K && !special) q = (int)rintf(ldexpf(x[k * xk], 23 - E)); // exact: |q| < 2^23
		int d0 = (int)(int8_t)(q & 255);
		int q1 = (q - d0) >> 8;
		int d1 = (int)(int8_t)(q1 & 255);
		int d2 = (q1 - d1) >> 8;
		int8_t *p = blk + (k >> 5) * 3072 + (((k >> 4) & 1) * 32 + r) * 16 + (k & 15);
		p[0] = (int8_t)d0;
		p[1024] = (int8_t)d1;
		p[2048] = (int8_t)d2;
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

// 16 int4 codes (8 packed bytes, see the layout above) as 16 int8 lanes of an MFMA operand
__device__ inline v4i unpack4(unsigned w0, unsigned w1)
{
	v4i r;
	r.x = (int)(w0 & 0x0f0f0f0fu);
	r.y = (int)(w1 & 0x0f0f0f0fu);
	r.z = (int)((w0 >> 4) & 0x0f0f0f0fu);
	r.w = (int)((w1 >> 4) & 0x0f0f0f0fu);
	return r;
}

__device__ inline void epilogue(const tgk_qgemm_args &a, const tgk_qweight &w, const Scratch &s, int Mp, int m, int c, int acc0,
				int acc1, int acc2, long corr)
{
	if (m >= a.M || c >= w.C) return;
	float acc32;
	if (s.special[m]) { // the reference's sequential loop (runtime/tg_rt.h:132-151)
		const float *x = xrow(a, m);
		float t = 0.0f;
		for (int k = 0; k < w.K; k++) t += (float)code_orig(w, c, k) * x[k * a.xk];
		acc32 = t;
	} else {
		long t0 = (long)acc0 - corr * s.sum[m];
		long t1 = (long)acc1 - corr * s.sum[Mp + m];
		long t2 = (long)acc2 - corr * s.sum[2 * Mp + m];
		long tot = t0 + t1 * 256 + t2 * 65536; // exact: |tot| < 2^53
		acc32 = (float)ldexp((double)tot, s.e[m] - 23);
	}
	int r = m / a.ni, jj = m - r * a.ni;
	a.o[(long)r * a.orr + (long)c * a.oc + (long)jj * a.oj] = w.scale[c] * acc32;
}

// s_waitcnt immediates (gfx9 encoding: vmcnt [3:0], expcnt [6:4], lgkmcnt [11:8]):
// wait until at most n vector-memory loads of this wave are outstanding and
// every LDS access has completed.
template <int N>
__device__ inline void wait_vm_lgkm0() { __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4)); }

// One 1 KiB global -> LDS copy by a wave: lane l moves 16 bytes from src to
// LDS address lds + 16 l. Issued with inline assembly so that the compiler,
// which cannot tell these copies apart from the LDS reads of other ring
// stages, does not drain all outstanding copies before every read; the K
// loop waits for exactly the stage it needs (wait_vm_lgkm0) instead.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ inline void copy_to_lds(const void *src, unsigned lds)
{
	asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop

// 512 threads = 8 waves; the workgroup computes a 128 x 128 tile (rows x
// channels), wave (wm, wn) a 32 x 64 block as two 32 x 32 blocks of
// v_mfma_i32_32x32x32_i8 for each of the three digit planes (96 accumulator
// registers). Each 64-input step needs 24 KiB of digits and 4 or 8 KiB of
// weights, copied by the waves straight from global memory into a ring of S
// LDS stages (global_load_lds, 1 KiB per wave instruction, no registers), so
// S - 1 steps are in flight while the waves multiply out of the oldest stage,
// with one barrier per step.
template <int BITS>
__global__ __launch_bounds__(512) void qgemm_k(tgk_qgemm_args a, tgk_qweight w, Scratch s, int Mp, int gx, int gy)
{
	constexpr int S = BITS == 4 ? 5 : 4;              // ring stages
	constexpr int AST = 24 * 1024;                   // 4 row blocks x 2 substeps x 3 digits x 1 KiB
	constexpr int BST = BITS == 4 ? 4096 : 8192;     // 4 channel blocks x 2 substeps x 512 B or 1 KiB
	constexpr int STG = AST + BST, NL = STG / 1024;   // 1 KiB wave copies per stage: 28 or 32
	constexpr int LW = 4;                            // copies per wave (wave 7 has none for int4)
	__shared__ __attribute__((aligned(1024))) uint8_t lds[S * STG];
	const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
	const int wm = wave & 3, wn = wave >> 2;
	// XCD-aware tile order: workgroups are dealt to the 8 XCDs round robin, so
	// renumber them to give each XCD a contiguous band of row tiles (its L2
	// then holds those rows' digits for every channel tile).
	int id = blockIdx.x, T = gx * gy;
	if (T % 8 == 0) id = (id % 8) * (T / 8) + id / 8;
	const int bm = id / gx, bn = id % gx;
	const int m0 = bm * BM, c0 = bn * BN, nk = w.Kp / KB, kblocks = w.Kp / 32;
	const uint8_t *gA = (const uint8_t *)s.dig + (long)(m0 / 32) * kblocks * 3072;
	const uint8_t *gB = w.w + (long)(c0 / 32) * kblocks * (BITS == 4 ? 512 : 1024);
	// this wave's copies: source at step 0 (lane offset included) and bytes per step
	const uint8_t *src0[LW];
	long sstep[LW];
	int nq = 0;
	for (int i = 0; i < LW; i++) {
		const int q = wave * LW + i;
		if (q >= NL) break;
		nq++;
		if (q < 24) {
			src0[i] = gA + (long)(q / 6) * kblocks * 3072 + (q % 6) * 1024;
			sstep[i] = 6144;
		} else if (BITS == 4) {
			src0[i] = gB + (long)(q - 24) * kblocks * 512;
			sstep[i] = 1024;
		} else {
			src0[i] = gB + (long)((q - 24) >> 1) * kblocks * 1024 + ((q - 24) & 1) * 1024;
			sstep[i] = 2048;
		}
		src0[i] += lane * 16;
	}
	const unsigned lds0 = (unsigned)(size_t)(__attribute__((address_space(3))) uint8_t *)lds;
	auto issue = [&](int kt) {
		const unsigned dst = lds0 + (unsigned)((kt % S) * STG + wave * LW * 1024);
		for (int i = 0; i < nq; i++) copy_to_lds(src0[i] + kt * sstep[i], __builtin_amdgcn_readfirstlane(dst + i * 1024));
	};
	v16i acc[3][2];
	for (int l = 0; l < 3; l++)
		for (int j = 0; j < 2; j++)
			for (int v = 0; v < 16; v++) acc[l][j][v] = 0;
	for (int st = 0; st < S - 1; st++)
		if (st < nk) issue(st);
	for (int kt = 0; kt < nk; kt++) {
		const int later = nk - 1 - kt < S - 2 ? nk - 1 - kt : S - 2; // stages issued after kt, maybe in flight
		if (nq == LW) { // a wave without copies has nothing to wait for
			switch (later) {
			case 0: wait_vm_lgkm0<0>(); break;
			case 1: wait_vm_lgkm0<LW>(); break;
			case 2: wait_vm_lgkm0<2 * LW>(); break;
			default: wait_vm_lgkm0<3 * LW>(); break;
			}
		} else {
			wait_vm_lgkm0<0>();
		}
		__builtin_amdgcn_sched_barrier(0);
		__builtin_amdgcn_s_barrier(); // stage kt is in LDS for every wave; stage kt - 1 is no longer read
		__builtin_amdgcn_sched_barrier(0);
		asm volatile("" ::: "memory"); // LDS changed behind the compiler's back: reload it
		if (kt + S - 1 < nk) issue(kt + S - 1);
		const uint8_t *A = lds + (kt % S) * STG, *B = A + AST;
		for (int kk = 0; kk < 2; kk++) {
			v4i af[3], bf[2];
			for (int l = 0; l < 3; l++) af[l] = *(const v4i *)(A + (wm * 6 + kk * 3 + l) * 1024 + lane * 16);
			for (int j = 0; j < 2; j++) {
				const int cb = wn * 2 + j;
				if (BITS == 4) {
					uint2 u = *(const uint2 *)(B + cb * 1024 + kk * 512 + lane * 8);
					bf[j] = unpack4(u.x, u.y);
				} else {
					bf[j] = *(const v4i *)(B + (cb * 2 + kk) * 1024 + lane * 16);
				}
			}
			for (int l = 0; l < 3; l++)
				for (int j = 0; j < 2; j++) acc[l][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[l], bf[j], acc[l][j], 0, 0, 0);
		}
	}
	const long corr = BITS == 4 ? 8 : 0;
	const int r32 = lane & 31, h = lane >> 5;
	for (int j = 0; j < 2; j++)
		for (int v = 0; v < 16; v++) // 32 x 32 accumulator: column lane % 32, row 8 (v / 4) + 4 (lane / 32) + v % 4
			epilogue(a, w, s, Mp, m0 + wm * 32 + 8 * (v >> 2) + 4 * h + (v & 3), c0 + wn * 64 + j * 32 + r32, acc[0][j][v], acc[1][j][v],
				 acc[2][j][v], corr);
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
	w->Cp = (int)round_up(C, BN);
	const int kblocks = w->Kp / 32, lb = bits == 8 ? 16 : 8; /* bytes per lane per 32-input block */
	size_t nb = (size_t)w->Cp * w->Kp * bits / 8, ob = bits == 8 ? (size_t)C * K : ((size_t)C * K + 1) / 2;
	uint8_t *h = (uint8_t *)calloc(nb, 1);
	float *hs = (float *)calloc((size_t)w->Cp, sizeof(float));
	if (!h || !hs) {
		free(h);
		free(hs);
		return -1;
	}
	if (bits == 4) memset(h, 0x88, nb); /* padding codes 0 */
	for (int c = 0; c < C; c++) {
		for (int k = 0; k < K; k++) {
			long i = axis == 0 ? (long)c * K + k : (long)k * C + c;
			int code;
			if (bits == 8) code = (signed char)codes[i];
			else {
				int b = (signed char)codes[i >> 1];
				code = (i & 1) ? (b >> 4) : (int)(signed char)(unsigned char)((unsigned)b << 4) >> 4;
			}
			const int lane = ((k >> 4) & 1) * 32 + (c & 31), kb = k & 15;
			uint8_t *frag = h + (((size_t)(c >> 5) * kblocks + (k >> 5)) * 64 + lane) * lb;
			if (bits == 8) {
				frag[kb] = (uint8_t)(int8_t)code;
			} else {
				unsigned t = (unsigned)(code + 8);
				uint8_t *byte = frag + (kb & 7);
				*byte = kb < 8 ? (uint8_t)((*byte & 0xf0) | t) : (uint8_t)((*byte & 0x0f) | (t << 4));
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
	long Mp = round_up(M, BM);
	return (size_t)Mp * Kp * 3 + (size_t)Mp * sizeof(int) * 5 + 256;
}

void tgk_qgemm_digits(hipStream_t st, const tgk_qgemm_args *a, void *scratch)
{
	const tgk_qweight *w = a->w;
	if (!w || !w->w || !a->x || !scratch || a->M <= 0 || a->ni <= 0) return; /* nothing valid to launch */
	int Mp = (int)round_up(a->M, BM);
	digits_k<<<Mp, 256, 0, st>>>(*a, carve(scratch, Mp, w->Kp), w->K, w->Kp, a->M);
}

void tgk_qgemm_mfma(hipStream_t st, const tgk_qgemm_args *a, void *scratch)
{
	const tgk_qweight *w = a->w;
	if (!w || !w->w || !w->scale || !a->x || !a->o || !scratch || a->M <= 0 || a->ni <= 0) return;
	int Mp = (int)round_up(a->M, BM);
	Scratch s = carve(scratch, Mp, w->Kp);
	int gx = w->Cp / BN, gy = Mp / BM;
	if (w->bits == 8) qgemm_k<8><<<gx * gy, 512, 0, st>>>(*a, *w, s, Mp, gx, gy);
	else qgemm_k<4><<<gx * gy, 512, 0, st>>>(*a, *w, s, Mp, gx, gy);
}

void tgk_qgemm(hipStream_t st, const tgk_qgemm_args *a, void *scratch)
{
	tgk_qgemm_digits(st, a, scratch);
	tgk_qgemm_mfma(st, a, scratch);
}
