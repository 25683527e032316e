// Quantized linear layers on the gfx950 int8 matrix cores.
//
// The reference computes o[c] = s[c] * (sum_k (float)code[c][k] * x[k]) with an
// f32 running sum (runtime/tg_rt.h:132-151). Here each activation row is
// written exactly as a 24-bit fixed-point vector q = rint(x * 2^(23-E)) with E
// the row's exponent (max |x| < 2^E), and q is split into three balanced int8
// digits q = d0 + 256 d1 + 65536 d2. v_mfma_i32_32x32x32_i8 sums code * d_l in
// int32 exactly for each digit l; the digit sums are combined in int64, scaled
// by 2^(E-23) in double (exact) and rounded to f32 once, then multiplied by
// the channel scale in f32 like the reference. The only approximation is the
// 24-bit activation grid (error <= 2^-24 max|x| per element), far below the
// reference's own f32 summation error at these K. Every step depends on the
// row alone, so a row's outputs do not depend on the batch it came in.
//
// Rows with a non-finite or huge entry are flagged by the digit kernel and
// their outputs are recomputed in the epilogue with the reference's exact
// sequential f32 loop, so inf/nan propagate as they do in the reference.
// Rows whose grid may be too coarse (a few entries far above the others,
// tg_qdigits.h) are flagged as candidates and resolved after the digit
// kernel (resolve_k) at every batch size: they keep their grid, or are split
// (outliers as exact terms, the rest on a grid of its own), or take the
// reference's loop, by a decision made from the row's values alone.
//
// Operand layouts in global memory are the MFMA fragment order of
// v_mfma_i32_32x32x32_i8 (lane l holds row or channel l % 32 and inputs
// 16 (l / 32) .. +15 of a 32-input block), so every fragment is one contiguous
// 1 KiB (or 512 B) block: the large-batch kernel copies them straight into LDS
// (global_load_lds_dwordx4) and the small-batch kernel straight into registers.
//   digits   [row / 32][k / 32][digit 0..2][lane 0..63][16 bytes]
//   int8 w   [channel / 32][k / 32][lane][16 codes]
//   int4 w   [channel / 32][k / 32][lane][8 bytes]: byte b holds t(b) in its
//            low nibble and t(b + 8) in its high nibble of the lane's 16
//            inputs, t = code + 8 in [0, 15] (offset binary), so unpacking is
//            two masks per 4 bytes; the +8 bias is removed with the row's sum
//            of q: sum_k t q = sum_k code q + 8 sum_k q.
//   int4 wg  (the large-batch kernel's copy) [channel / 64][k / 32][lane][16
//            bytes]: byte b of lane l holds, for input 16 (l / 32) + b of the
//            block, t = code + 8 of channel l % 32 of the pair's first 32 in its
//            low nibble and the code (two's complement) of channel 32 + l % 32
//            in its high nibble. As an int8 the byte is t + 16 code', so the
//            raw bytes are one MFMA operand (sums S1 = sum t q + 16 sum code' q)
//            and the bytes masked to their low nibbles another (S0 = sum t q):
//            the second channel's sum is (S1 - S0) / 16, exactly, with one mask
//            per 4 bytes for two channel blocks instead of three operations
//            per 4 bytes for each.
// Weights are repacked once at load (channels padded to 256, K to 64).
#include "tg_ewop.h"
#include "tg_kern.h"
#include "tg_qdigits.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <type_traits>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

namespace {

constexpr int KB = 64;        // K padding (one K step of the LDS kernel)
constexpr int BM = 128;       // rows per tile of the LDS kernel (activation rows are padded to it)
constexpr int DEFER_RESOLVE_ROWS = 131072; // digit batches from which candidates are resolved by a pass of their own
constexpr int BN = 256;       // channels per tile of the LDS kernel (weights are padded to it)

inline long round_up(long x, long m) { return (x + m - 1) / m * m; }

struct Scratch {
	int8_t *dig;       // digits in fragment order (see above)
	long long *qsum;   // [Mp] sum over k of the row's fixed-point values q
	int *e;            // [Mp] row exponent E
	int *special;      // [Mp] 0 a grid row; 1 the reference's sequential loop (or a candidate before resolve_k); 2 a split row
	int *ok;           // [Mp][tgq_nout(Kp)] a split row's outliers: input index, -1 past the last
	float *ox;         // [Mp][tgq_nout(Kp)] and value
};

Scratch carve(void *base, int Mp, int Kp)
{
	Scratch s;
	char *p = (char *)base;
	s.dig = (int8_t *)p;
	p += (size_t)Mp * Kp * 3; // Kp is a multiple of 64: 8-byte alignment holds
	s.qsum = (long long *)p;
	p += (size_t)Mp * sizeof(long long);
	s.e = (int *)p;
	p += (size_t)Mp * sizeof(int);
	s.special = (int *)p;
	p += (size_t)Mp * sizeof(int);
	s.ok = (int *)p;
	p += (size_t)Mp * tgq_nout(Kp) * sizeof(int);
	s.ox = (float *)p;
	return s;
}

// element 0 of activation row m
__device__ inline const float *xrow(const tgk_qgemm_args &a, int m)
{
	int r = m / a.ni, j = m - r * a.ni;
	return a.x + (long)r * a.xr + (long)j * a.xj;
}

__device__ inline float wave_max(float v)
{
	for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
	return v;
}

__device__ inline long long wave_sum(long long v)
{
	for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
	return v;
}

// inputs k0 .. k0 + 15 of a row. The addresses are clamped into the row
// instead of branched on, so the loads of several calls can all be in flight
// before the first value is used. vec (unit stride, 16-byte aligned row, K a
// multiple of 16, so whole float4s): a group at or past K reads the row's
// first 16 inputs instead, which leave the row's max and NaN flag unchanged;
// the caller writes such a group as zero digits (tgq_put16's `zero`).
// Otherwise inputs at and beyond K read as zeros.
template <bool VEC>
__device__ inline void load16(float *v, const float *x, long xk, int k0, int K)
{
	if (VEC) {
		const float *p = x + (k0 < K ? k0 : 0);
		for (int i = 0; i < 4; i++) {
			const float4 f = *(const float4 *)(p + 4 * i);
			v[4 * i] = f.x, v[4 * i + 1] = f.y, v[4 * i + 2] = f.z, v[4 * i + 3] = f.w;
		}
	} else {
		for (int i = 0; i < 16; i++) {
			const int k = k0 + i;
			const float f = x[(long)(k < K ? k : K - 1) * xk];
			v[i] = k < K ? f : 0.0f;
		}
	}
}

// One wave per activation row (4 rows per block): exponent, digits, sum of q,
// special flag. Lane l owns inputs 1024 s + 16 l .. +15 of each 1024-input
// slab s. Rows of up to SL slabs are read once into registers; longer rows are
// read twice (max, then digits), the second time from cache.
template <int SL>
__global__ __launch_bounds__(256) void digits_k(tgk_qgemm_args a, Scratch s, int K, int Kp, int M)
{
	const int lane = threadIdx.x & 63;
	const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
	if (m >= M) return; // the whole wave leaves; the kernel has no block barrier
	const float *x = xrow(a, m);
	const long xk = a.xk;
	const bool vec = xk == 1 && ((size_t)x & 15) == 0 && (K & 15) == 0;
	const int nsl = (Kp + 1023) / 1024;
	float v[SL][16];
	unsigned mb = 0; // max |x| as bits (tgq_scan16)
	// slabs t0 .. t0 + SL - 1 into v, loads first; slabs past the row read as
	// zeros (no branch, so every load is in flight before the first use)
	auto fetch = [&](int t0) {
		if (vec)
			for (int t = 0; t < SL; t++) load16<true>(v[t], x, xk, (t0 + t) * 1024 + lane * 16, K);
		else
			for (int t = 0; t < SL; t++) load16<false>(v[t], x, xk, (t0 + t) * 1024 + lane * 16, K);
	};
	for (int t0 = 0; t0 < nsl; t0 += SL) {
		fetch(t0);
		for (int t = 0; t < SL; t++)
			tgq_scan16(v[t], mb);
	}
	float mx;
	int bad;
	tgq_scan_end(mb, mx, bad);
	const float amax = wave_max(mx); // a NaN lane reads 0 here; its row is flagged by `bad`
	const int special = tgq_special(__any(bad), amax), E = tgq_exponent(amax, special);
	long long qs = 0, tl = 0;
	int8_t *blk = tgq_row_base(s.dig, m, Kp);
	for (int t0 = 0; t0 < nsl; t0 += SL) {
		if (nsl > SL) fetch(t0); // rows of up to SL slabs are still in v
		for (int t = 0; t < SL; t++) {
			const int k0 = (t0 + t) * 1024 + lane * 16;
			if (t0 + t < nsl && k0 < Kp) qs += tgq_put16(blk, k0, v[t], E, special || k0 >= K, tl);
		}
	}
	qs = wave_sum(qs);
	tl = wave_sum(tl);
	int cls = special ? TGQ_REF : tgq_candidate(tl) ? TGQ_CAND : TGQ_GRID;
	if (cls == TGQ_CAND) { // the coarse test first (the row again: still in v when it fits, else read again)
		TgqCoarse co{};
		for (int t0 = 0; t0 < nsl; t0 += SL) {
			if (nsl > SL) fetch(t0);
			for (int t = 0; t < SL; t++) {
				const int k0 = (t0 + t) * 1024 + lane * 16;
				if (t0 + t < nsl && k0 < K) tgq_coarse16(co, v[t], E);
			}
		}
		if (tgq_coarse_grid(tgq_coarse_wave_sum(co), tl)) cls = TGQ_GRID;
	}
	if (lane == 0) {
		s.e[m] = E;
		s.special[m] = cls;
		s.qsum[m] = qs;
	}
	if (cls == TGQ_CAND) { // this wave wrote the row's digits (lane l its groups l + 64 j): it resolves the row
		__shared__ TgqHist hist[4];
		const int nout = tgq_nout(Kp);
		auto ld = [&](int g, float *v) {
			if (g * 16 >= K)
				for (int i = 0; i < 16; i++) v[i] = 0.0f;
			else if (vec) load16<true>(v, x, xk, g * 16, K);
			else load16<false>(v, x, xk, g * 16, K);
		};
		tgq_resolve_row(&hist[threadIdx.x >> 6], ld, K, Kp, E, blk, &s.qsum[m], &s.e[m], &s.special[m], s.ok + (long)m * nout,
				s.ox + (long)m * nout, nout, lane);
	}
}

// Many rows, 16 per block: lane l of wave w owns row m0 + (l & 15), half
// (l >> 4) & 1 and parity l >> 5 of 32-input block pairs w, w + W, ... (NKB
// pairs in registers). In each digit plane a block writes its 16 rows' two
// 256-byte runs. A row's max, non-finite flag, sum of q and tallies are
// combined over its four lanes of a wave with shuffles, then over the waves
// through LDS. Candidates take the coarse test on the values still in
// registers; those it does not settle are resolved a wave per row by the
// first RW waves, whose histograms are the dynamic LDS (RW x TgqHist). Results
// are those of digits_k.
template <int NKB, bool VEC>
__global__ __launch_bounds__(1024) void digits_tile16_k(tgk_qgemm_args a, Scratch s, int K, int Kp, int M, int RW)
{
	__shared__ float smx[16][16];
	__shared__ int sbad[16][16];
	__shared__ long long sqs[16][16], stl[16][16];
	__shared__ TgqCoarse sco[16][16];
	__shared__ int scls[16], sE[16], sany;
	extern __shared__ TgqHist hist[];
	const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, W = blockDim.x >> 6;
	const int m0 = blockIdx.x * 16, mr = lane & 15, half = (lane >> 4) & 1, par = lane >> 5;
	const float *x = xrow(a, m0 + mr < M ? m0 + mr : M - 1); // rows past M repeat row M - 1
	const int nkb = Kp / 32;
	float v[NKB][16];
	unsigned mb = 0; // max |x| as bits (tgq_scan16)
	for (int j = 0; j < NKB; j++) {
		const int kb = 2 * (w + j * W) + par;
		load16<VEC>(v[j], x, a.xk, kb < nkb ? kb * 32 + half * 16 : K, K); // past the row: zeros
		tgq_scan16(v[j], mb);
	}
	float mx;
	int bad;
	tgq_scan_end(mb, mx, bad);
	for (int o = 16; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o)), bad |= __shfl_xor(bad, o);
	if (lane < 16) smx[w][lane] = mx, sbad[w][lane] = bad;
	__syncthreads();
	float amax = 0.0f;
	bad = 0;
	for (int u = 0; u < W; u++) amax = fmaxf(amax, smx[u][mr]), bad |= sbad[u][mr];
	const int special = tgq_special(bad, amax), E = tgq_exponent(amax, special);
	int8_t *blk = s.dig + (long)(m0 >> 5) * nkb * 3072 + ((m0 & 31) + mr) * 16;
	long long qs = 0, tl = 0;
	for (int j = 0; j < NKB; j++) {
		const int kb = 2 * (w + j * W) + par;
		if (kb < nkb) qs += tgq_put16(blk, kb * 32 + half * 16, v[j], E, special || kb * 32 + half * 16 >= K, tl);
	}
	for (int o = 16; o < 64; o <<= 1) qs += __shfl_xor(qs, o), tl += __shfl_xor(tl, o);
	if (lane < 16) sqs[w][lane] = qs, stl[w][lane] = tl;
	__syncthreads(); // also: every digit of the block's rows is stored
	if (w == 0 && lane < 16) {
		long long t = 0, u2 = 0;
		for (int u = 0; u < W; u++) t += sqs[u][mr], u2 += stl[u][mr];
		const int cls = m0 + mr >= M ? TGQ_GRID : special ? TGQ_REF : tgq_candidate(u2) ? TGQ_CAND : TGQ_GRID;
		scls[mr] = cls, sE[mr] = E;
		stl[0][mr] = u2; // the row's tally, for the coarse test
		if (m0 + mr < M) s.e[m0 + mr] = E, s.special[m0 + mr] = cls, s.qsum[m0 + mr] = t;
		const unsigned long long cb = __ballot(cls == TGQ_CAND);
		if (lane == 0) sany = cb != 0;
	}
	__syncthreads();
	if (!sany) return; // (uniform over the block)
	// the coarse test of the candidates, on the values still in registers
	TgqCoarse co{};
	if (scls[mr] == TGQ_CAND)
		for (int j = 0; j < NKB; j++) {
			const int kb = 2 * (w + j * W) + par;
			if (kb < nkb && kb * 32 + half * 16 < K) tgq_coarse16(co, v[j], E);
		}
	for (int o = 16; o < 64; o <<= 1)
		co.cnt += __shfl_xor(co.cnt, o), co.s0 += __shfl_xor(co.s0, o), co.s1 += __shfl_xor(co.s1, o);
	if (lane < 16) sco[w][lane] = co;
	__syncthreads();
	if (w == 0 && lane < 16 && scls[mr] == TGQ_CAND) {
		TgqCoarse c = sco[0][mr];
		for (int u = 1; u < W; u++) tgq_coarse_add(c, sco[u][mr]);
		if (tgq_coarse_grid(c, stl[0][mr])) {
			scls[mr] = TGQ_GRID;
			s.special[m0 + mr] = TGQ_GRID;
		}
	}
	__syncthreads();
	// the rest of the candidates: a wave per row (waves 0 .. RW - 1), each row read again
	const int nout = tgq_nout(Kp);
	if (w < RW)
		for (int r = w; r < 16; r += RW) {
			if (scls[r] != TGQ_CAND) continue;
			const int m = m0 + r;
			const float *xr = xrow(a, m);
			auto ld = [&](int g, float *v) {
				if (g * 16 >= K)
					for (int i = 0; i < 16; i++) v[i] = 0.0f;
				else load16<VEC>(v, xr, a.xk, g * 16, K);
			};
			tgq_resolve_row(&hist[w], ld, K, Kp, sE[r], tgq_row_base(s.dig, m, Kp), &s.qsum[m], &s.e[m], &s.special[m], s.ok + (long)m * nout,
					s.ox + (long)m * nout, nout, lane);
		}
}

// Row m's digits and row data made by one workgroup of NW waves, thread t
// taking the 16-input groups t, t + 64 NW, ... (G of them, in registers). The
// row's max, non-finite flag and sum of q are combined across the workgroup.
// Results are those of digits_k.
template <int NW, int G, bool VEC>
__device__ inline void row_digits(const tgk_qgemm_args &a, const Scratch &s, int K, int Kp, int m)
{
	constexpr int NT = 64 * NW;
	__shared__ float smx[NW];
	__shared__ int sbad[NW];
	__shared__ long long sqs[NW], stl[NW];
	const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, ng = Kp / 16;
	const float *x = xrow(a, m);
	float v[G][16];
	unsigned mb = 0; // max |x| as bits (tgq_scan16)
	for (int g = 0; g < G; g++) {
		const int j = tid + g * NT;
		load16<VEC>(v[g], x, a.xk, j < ng ? j * 16 : K, K); // past the row: zeros
		tgq_scan16(v[g], mb);
	}
	float mx;
	int bad;
	tgq_scan_end(mb, mx, bad);
	mx = wave_max(mx); // a NaN lane reads 0 here; its row is flagged by `bad`
	bad = __any(bad);
	if (lane == 0) smx[w] = mx, sbad[w] = bad;
	__syncthreads();
	float amax = smx[0];
	int anybad = sbad[0];
	for (int u = 1; u < NW; u++) amax = fmaxf(amax, smx[u]), anybad |= sbad[u];
	const int special = tgq_special(anybad, amax), E = tgq_exponent(amax, special);
	int8_t *blk = tgq_row_base(s.dig, m, Kp);
	long long qs = 0, tl = 0;
	for (int g = 0; g < G; g++) {
		const int j = tid + g * NT;
		if (j < ng) qs += tgq_put16(blk, j * 16, v[g], E, special || j * 16 >= K, tl);
	}
	qs = wave_sum(qs);
	tl = wave_sum(tl);
	if (lane == 0) sqs[w] = qs, stl[w] = tl;
	__syncthreads(); // also: every digit of the row is stored
	long long tally = 0, qsum = 0;
	for (int u = 0; u < NW; u++) tally += stl[u], qsum += sqs[u];
	int cls = special ? TGQ_REF : tgq_candidate(tally) ? TGQ_CAND : TGQ_GRID;
	if (cls == TGQ_CAND) { // (uniform over the block) the coarse test, on the values still in registers
		__shared__ TgqCoarse sco[NW];
		TgqCoarse co{};
		for (int g = 0; g < G; g++) {
			const int j = tid + g * NT;
			if (j < ng && j * 16 < K) tgq_coarse16(co, v[g], E);
		}
		co = tgq_coarse_wave_sum(co);
		if (lane == 0) sco[w] = co;
		__syncthreads();
		TgqCoarse c = sco[0];
		for (int u = 1; u < NW; u++) tgq_coarse_add(c, sco[u]);
		if (tgq_coarse_grid(c, tally)) cls = TGQ_GRID;
	}
	if (tid == 0) {
		s.e[m] = E;
		s.special[m] = cls;
		s.qsum[m] = qsum;
	}
	if (cls == TGQ_CAND && w == 0) { // wave 0 resolves the row (uniform: cls is the block's)
		__shared__ TgqHist hist;
		const int nout = tgq_nout(Kp);
		auto ld = [&](int g, float *v) {
			if (g * 16 >= K)
				for (int i = 0; i < 16; i++) v[i] = 0.0f;
			else load16<VEC>(v, x, a.xk, g * 16, K);
		};
		tgq_resolve_row(&hist, ld, K, Kp, E, blk, &s.qsum[m], &s.e[m], &s.special[m], s.ok + (long)m * nout, s.ox + (long)m * nout, nout,
				lane);
	}
}

// Few, long rows: one block of 256 threads per row (row_digits)
template <int G, bool VEC>
__global__ __launch_bounds__(256) void digits_row_k(tgk_qgemm_args a, Scratch s, int K, int Kp, int M)
{
	row_digits<4, G, VEC>(a, s, K, Kp, blockIdx.x);
}

// Candidate rows (tg_qdigits.h) of a digit area whose producer did not
// resolve them (the decoder's fused producers): a wave per row
// (tgq_resolve_row, the digit kernels' own resolve), rows of other classes
// left as they are. Wave v takes rows v, v + (total waves), ...
template <bool VEC>
__global__ __launch_bounds__(256) void resolve_k(tgk_qgemm_args a, Scratch s, int K, int Kp, int M)
{
	__shared__ TgqHist hist[4];
	const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nout = tgq_nout(Kp);
	// a wave reads the classes of 16 rows at once (a lane each) and resolves
	// that group's candidates one after another, so a batch with few
	// candidates costs a few loads per wave, not one dependent load per row
	for (long m0 = ((long)blockIdx.x * 4 + wave) * 16; m0 < M; m0 += (long)gridDim.x * 64) {
		unsigned long long cb = __ballot(lane < 16 && m0 + lane < M && s.special[m0 + lane] == TGQ_CAND);
		while (cb) {
			const long m = m0 + __builtin_ctzll(cb);
			cb &= cb - 1;
			const float *x = xrow(a, (int)m);
			auto ld = [&](int g, float *v) {
				if (g * 16 >= K)
					for (int i = 0; i < 16; i++) v[i] = 0.0f;
				else load16<VEC>(v, x, a.xk, g * 16, K);
			};
			tgq_resolve_row(&hist[wave], ld, K, Kp, s.e[m], tgq_row_base(s.dig, (int)m, Kp), &s.qsum[m], &s.e[m], &s.special[m],
					s.ok + m * nout, s.ox + m * nout, nout, lane);
		}
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

// digit sums -> sum_k t q (exact: |.| < 2^53)
__device__ inline long long combine(int acc0, int acc1, int acc2)
{
	return (long long)acc0 + (long long)acc1 * 256 + (long long)acc2 * 65536;
}

// the same sum in f64, also exact: every term and partial sum is an integer
// below 2^48 in magnitude (int32 digit sums times at most 2^16), so each fused
// multiply-add gives the same value as a multiply then an add, in one
// instruction
__device__ inline double combine_d(int acc0, int acc1, int acc2)
{
	return __builtin_fma((double)acc2, 65536.0, __builtin_fma((double)acc1, 256.0, (double)acc0));
}

// output (m, c) from tot = sum_k t[c][k] q[m][k]
// output column c: its segment's base (shifted to the column) and row strides
struct OutCol {
	float *p;
	long orr, oj;
};
__device__ inline OutCol out_col(const tgk_qgemm_args &a, int c)
{
	if (a.nseg <= 1) return OutCol{ a.o + (long)c * a.oc, a.orr, a.oj };
	int g = 0;
	while (g + 1 < a.nseg && c >= a.seg_c0[g + 1]) g++;
	return OutCol{ a.seg_o[g] + (long)(c - a.seg_c0[g]) * a.oc, a.seg_orr[g], a.seg_oj[g] };
}

__device__ inline float *out_at(const tgk_qgemm_args &a, int r, int jj, int c)
{
	const OutCol o = out_col(a, c);
	return o.p + (long)r * o.orr + (long)jj * o.oj;
}

// a unary instruction of an epilogue chain, as the elementwise kernels compute it
__device__ inline float epi_uop(int op, float v) { return tg_uop(op, v); }

// output (batch row r, inner row jj, channel c) with value v (the product)
// after the epilogue chain: the values the instructions after the product
// would compute from it, one after another
__device__ inline float finish(const tgk_qgemm_args &a, int r, int jj, int c, float v)
{
	for (int e = 0; e < a.nepi; e++) {
		const tgk_epi &E = a.epi[e];
		if (E.kind == TGK_EW_UN) {
			v = epi_uop(E.op, v);
			continue;
		}
		const float *p = E.x + (long)r * E.xr;
		const float x = E.mode == 0 ? p[(long)jj * a.oj + (long)c * a.oc] : E.mode == 1 ? p[0] : p[c];
		v = E.kind == TGK_EW_BIN ? tg_bop(E.op, v, x) : tg_bop(E.op, x, v);
	}
	return v;
}

// the reference's sequential loop for output (m, c) (runtime/tg_rt.h:132-151)
__device__ inline float ref_loop(const tgk_qgemm_args &a, const tgk_qweight &w, int m, int c)
{
	const float *x = xrow(a, m);
	float t = 0.0f;
	for (int k = 0; k < w.K; k++) t += (float)code_orig(w, c, k) * x[k * a.xk];
	return t;
}

// The reference's sums of ref_loop for line m and channels c = cb + NQ lane
// + q (q < NQ), a whole wave on one line: the line's inputs have one address
// for every lane (read four at a time when they are contiguous), and the
// codes of U inputs are loaded before their multiplies and adds, which keep
// each sum's order; a lane's NQ channels are adjacent, so for weights stored
// [K][C] in int8 (x @ W) an input's NQ codes are one load. Channels at or
// beyond C read channel C - 1 and are not to be used.
// (VEC false: the plain loads only, for kernels with few registers to spare)
template <int NQ, int U = 16, bool VEC = true>
__device__ inline void ref_line(const tgk_qgemm_args &a, const tgk_qweight &w, int m, int cb, int lane, float (&t)[NQ])
{
	static_assert(U % 4 == 0 && (NQ == 1 || NQ == 2 || NQ == 4), "ref_line shape");
	const float *x = xrow(a, m);
	int c[NQ];
	for (int q = 0; q < NQ; q++) {
		const int cc = cb + NQ * lane + q;
		c[q] = cc < w.C ? cc : w.C - 1;
		t[q] = 0.0f;
	}
	const int K = w.K, c0 = cb + NQ * lane;
	// one load of the NQ codes of input k: int8, [K][C], the NQ channels in range and aligned
	const bool row8 = VEC && w.bits == 8 && w.axis == 1 && c0 + NQ <= w.C && (w.C % NQ) == 0 && ((size_t)w.orig % 4) == 0;
	const bool xv4 = VEC && a.xk == 1 && ((size_t)x % 16) == 0;
	int k = 0;
	for (; k + U <= K; k += U) {
		float xv[U];
		int cd[NQ][U];
		if (xv4)
			for (int u = 0; u < U; u += 4) {
				const float4 f = *(const float4 *)(x + k + u);
				xv[u] = f.x, xv[u + 1] = f.y, xv[u + 2] = f.z, xv[u + 3] = f.w;
			}
		else
			for (int u = 0; u < U; u++) xv[u] = x[(long)(k + u) * a.xk];
		if (row8)
			for (int u = 0; u < U; u++) {
				const int8_t *p = (const int8_t *)w.orig + (long)(k + u) * w.C + c0;
				if constexpr (NQ == 4) {
					const int v = *(const int *)p;
					for (int q = 0; q < 4; q++) cd[q][u] = (int)(int8_t)(v >> (8 * q));
				} else if constexpr (NQ == 2) {
					const short v = *(const short *)p;
					cd[0][u] = (int)(int8_t)v, cd[1][u] = (int)(int8_t)(v >> 8);
				} else
					cd[0][u] = p[0];
			}
		else
			for (int q = 0; q < NQ; q++)
				for (int u = 0; u < U; u++) cd[q][u] = code_orig(w, c[q], k + u);
		for (int u = 0; u < U; u++)
			for (int q = 0; q < NQ; q++) t[q] += (float)cd[q][u] * xv[u];
	}
	for (; k < K; k++) {
		const float xk = x[(long)k * a.xk];
		for (int q = 0; q < NQ; q++) t[q] += (float)code_orig(w, c[q], k) * xk;
	}
}

// output (m, c) from tot = sum_k t[c][k] q[m][k], given row m's exponent, special flag and sum of q
// ACT: TGM_TANH or TGM_SILU when that activation, read only by the product,
// is applied here (the chain [tanh] or [silu] of the large-batch kernel,
// inline), else 0
template <int ACT = 0>
__device__ inline float act_out(float v) { return ACT ? tg_uop(ACT, v) : v; }

// A split row's outlier terms for channel c (m < M, c < C): sum over its
// outliers, in increasing input order, of code[c][k] x_k in f64 (each
// product exact), from 0.0
__device__ inline double outlier_sum(const Scratch &s, const tgk_qweight &w, int m, int c)
{
	const int nout = tgq_nout(w.Kp);
	double t = 0.0;
	for (int j = 0; j < nout; j++) {
		const int k = s.ok[(long)m * nout + j];
		if (k < 0) break;
		t += (double)code_orig(w, c, k) * (double)s.ox[(long)m * nout + j];
	}
	return t;
}

// special: 0 a grid row, 1 the reference's loop, 2 a split row (the grid
// sum of its other entries plus its outliers' terms, in f64, rounded once)
// (sc: channel c's scale, read beforehand by callers that gather their loads)
template <int ACT = 0>
__device__ inline void epilogue_sc(const tgk_qgemm_args &a, const tgk_qweight &w, const Scratch &s, int m, int c, long long tot, int E,
				   int special, long long qsum, float sc)
{
	if (m >= a.M || c >= w.C) return;
	float acc32;
	if (special & 1) { // the reference's sequential loop (TGQ_REF, or a candidate no resolve has seen)
		acc32 = ref_loop(a, w, m, c);
	} else {
		if (w.bits == 4) tot -= 8 * qsum;
		const double g = ldexp((double)tot, E - 23);
		acc32 = (float)(special == 2 ? g + outlier_sum(s, w, m, c) : g);
	}
	int r = m / a.ni, jj = m - r * a.ni;
	*out_at(a, r, jj, c) = act_out<ACT>(sc * acc32);
}

template <int ACT = 0>
__device__ inline void epilogue_with(const tgk_qgemm_args &a, const tgk_qweight &w, const Scratch &s, int m, int c, long long tot,
				     int E, int special, long long qsum)
{
	if (m >= a.M || c >= w.C) return;
	epilogue_sc<ACT>(a, w, s, m, c, tot, E, special, qsum, w.scale[c]);
}

__device__ inline void epilogue(const tgk_qgemm_args &a, const tgk_qweight &w, const Scratch &s, int m, int c, long long tot)
{
	if (m >= a.M || c >= w.C) return;
	epilogue_with(a, w, s, m, c, tot, s.e[m], s.special[m], s.qsum[m]);
}

// One lane's outputs of a 32-row block: rows mbase + 8 (v / 4) + 4 (lane / 32)
// + v % 4 (v = 0 .. 15, the 32 x 32 accumulator layout) for NB column blocks
// cbase + 32 j + lane % 32; tot(j, v) gives sum_k t q. A wave without a
// special row (the common case) takes a straight-line path that reads each
// row's exponent and sum once and each column's scale once; otherwise every
// output goes through epilogue().
// What a lane's epilogue reads besides its sums: row mbase + lane % 32's
// exponent, sum of q and special flag, and the scales of its columns, all in
// one round trip; a lane's 16 rows then come from the lanes that hold them
// (shuffles), not from 16 dependent loads. A kernel may fetch it before its
// K loop, so that the loads' latency is hidden behind the loop.
template <int NB>
struct TileRows {
	int Er, spr;
	long long Qr;
	float sc[NB];
};
template <int NB>
__device__ inline TileRows<NB> tile_rows(const tgk_qgemm_args &a, const tgk_qweight &w, const Scratch &s, int mbase, int cbase, int lane)
{
	TileRows<NB> t;
	const int r32 = lane & 31, mr = mbase + r32, mrc = mr < a.M ? mr : a.M - 1;
	t.Er = s.e[mrc];
	t.spr = mr < a.M ? s.special[mrc] : 0;
	t.Qr = w.bits == 4 ? s.qsum[mrc] : 0;
	for (int j = 0; j < NB; j++) {
		const int c = cbase + j * 32 + r32;
		t.sc[j] = w.scale[c < w.Cp ? c : 0]; // scales are padded to Cp; columns at or beyond C are not written
	}
	return t;
}

// HOIST: take all 16 rows' exponents and sums of q from their lanes before the
// first store (the shuffles then wait once, not once per row; 48 more live
// registers, for kernels that have them free at the epilogue).
// W8: the weights are int8 (no +8 bias to take out, the sums of q unused),
// known when the kernel is compiled.
template <int NB, bool HOIST, int ACT = 0, bool PAIRS = false, bool W8 = false, class Tot, class TotD>
__device__ inline void store_tile(const tgk_qgemm_args &a, const tgk_qweight &w, const Scratch &s, int mbase, int cbase, int lane,
				  const TileRows<NB> &t, Tot tot, TotD totd)
{
	const int r32 = lane & 31, h = lane >> 5;
	const int Er = t.Er, spr = t.spr;
	const long long Qr = t.Qr;
	const float *sc = t.sc;
	int Ev[HOIST ? 16 : 1];
	long long Qv[HOIST ? 16 : 1];
	if constexpr (HOIST)
		for (int v = 0; v < 16; v++) {
			const int rv = 8 * (v >> 2) + 4 * h + (v & 3);
			Ev[v] = __shfl(Er, rv);
			Qv[v] = __shfl(Qr, rv);
		}
	auto row_e = [&](int v, int rv) { if constexpr (HOIST) return Ev[v]; else return __shfl(Er, rv); };
	auto row_q = [&](int v, int rv) { if constexpr (HOIST) return Qv[v]; else return __shfl(Qr, rv); };
	if (__any(spr)) { // rows of the reference's loop and split rows: the others as usual, each reference-loop row by the whole wave
		for (int v = 0; v < 16; v++) {
			const int rv = 8 * (v >> 2) + 4 * h + (v & 3), m = mbase + rv;
			const int E = __shfl(Er, rv), sp = __shfl(spr, rv);
			const long long Q = __shfl(Qr, rv);
			if (!(sp & 1))
				for (int j = 0; j < NB; j++) // a pair's odd block has no +8 bias to remove: add it for epilogue_with
					epilogue_with<ACT>(a, w, s, m, cbase + j * 32 + r32, tot(j, v) + (PAIRS && (j & 1) ? 8 * Q : 0), E, sp, Q);
		}
		unsigned long long sm = __ballot(spr & 1) & 0xffffffffull; // lane r (r < 32): row mbase + r
		while (sm) {
			const int rv = __builtin_ctzll(sm);
			sm &= sm - 1;
			const int m = mbase + rv;
			if (m >= a.M) continue;
			constexpr int NQ = (NB * 32 + 63) / 64;
			float t[NQ];
			ref_line<NQ, 4, false>(a, w, m, cbase, lane, t); // few registers: the accumulators may still be live
			const int r = m / a.ni, jj = m - r * a.ni;
			for (int q = 0; q < NQ; q++) {
				const int c = cbase + NQ * lane + q;
				if (c < cbase + NB * 32 && c < w.C) *out_at(a, r, jj, c) = act_out<ACT>(w.scale[c] * t[q]);
			}
		}
		return;
	}
	if (a.nseg > 1) { // a merged GEMM: each column's own output
		OutCol oc[NB];
		for (int j = 0; j < NB; j++) {
			const int c = cbase + j * 32 + r32;
			oc[j] = out_col(a, c < w.C ? c : 0);
		}
		// a whole block whose lines are evenly spaced in every column's
		// output: each column's row at its own base plus the row offset times
		// its own line stride, the loop unrolled, no bounds to test
		bool even = a.oc == 1 && mbase + 32 <= a.M && cbase + NB * 32 <= w.C;
		for (int j = 0; j < NB; j++) even = even && (a.ni == 1 || oc[j].orr == (long)a.ni * oc[j].oj);
		if (__all(even)) {
			float *pb[NB];
			long lsj[NB];
			for (int j = 0; j < NB; j++) {
				lsj[j] = a.ni == 1 ? oc[j].orr : oc[j].oj;
				pb[j] = oc[j].p + (long)(mbase + 4 * h) * lsj[j];
			}
			__builtin_amdgcn_s_waitcnt(0x0f70); // vmcnt(0): the row data and scales, once
#pragma unroll
			for (int v = 0; v < 16; v++) {
				const int dv = 8 * (v >> 2) + (v & 3), rv = dv + 4 * h;
				const int E = row_e(v, rv);
				const double q8 = W8 ? 0.0 : 8.0 * (double)row_q(v, rv);
#pragma unroll
				for (int j = 0; j < NB; j++) {
					const double tj = W8 || (PAIRS && (j & 1)) ? totd(j, v) : totd(j, v) - q8;
					pb[j][(long)dv * lsj[j]] = sc[j] * (float)ldexp(tj, E - 23); // no chain
				}
			}
			return;
		}
		for (int v = 0; v < 16; v++) {
			const int rv = 8 * (v >> 2) + 4 * h + (v & 3), m = mbase + rv;
			const int E = row_e(v, rv);
			const double q8 = 8.0 * (double)row_q(v, rv); // 0 for int8 weights
			if (m >= a.M) continue;
			int r = m, jj = 0;
			if (a.ni != 1) r = m / a.ni, jj = m - r * a.ni;
			for (int j = 0; j < NB; j++) {
				if (cbase + j * 32 + r32 >= w.C) continue;
				oc[j].p[(long)r * oc[j].orr + (long)jj * oc[j].oj] =
					sc[j] * (float)ldexp(totd(j, v) - (PAIRS && (j & 1) ? 0.0 : q8), E - 23); // no chain
			}
		}
		return;
	}
	// line m's output row at a.o + m ls (lines evenly spaced: one per batch
	// row, or inner rows packed ni to a batch row)
	const long ls = a.ni == 1 ? a.orr : a.oj;
	if (a.oc == 1 && (a.ni == 1 || a.orr == (long)a.ni * a.oj) && mbase + 32 <= a.M && cbase + NB * 32 <= w.C) {
		// a whole block (its 32 rows and NB x 32 columns exist) of evenly
		// spaced lines, channels at stride 1: a lane's rows at its base plus a
		// wave-uniform offset, its columns at fixed offsets from the row; the
		// loop unrolled, so every sum is read from its own register, and no
		// bounds to test
		float *ob = a.o + (long)(mbase + 4 * h) * ls + cbase + r32;
		// the row data and scales have landed: one wait here, not one in
		// front of a store after each branch that skips a store
		__builtin_amdgcn_s_waitcnt(0x0f70); // vmcnt(0)
#pragma unroll
		for (int v = 0; v < 16; v++) {
			const int dv = 8 * (v >> 2) + (v & 3), rv = dv + 4 * h;
			const int E = row_e(v, rv);
			const double q8 = W8 ? 0.0 : 8.0 * (double)row_q(v, rv);
			float *orow = ob + (long)dv * ls;
#pragma unroll
			for (int j = 0; j < NB; j++) {
				const double tj = W8 || (PAIRS && (j & 1)) ? totd(j, v) : totd(j, v) - q8;
				orow[32 * j] = act_out<ACT>(sc[j] * (float)ldexp(tj, E - 23));
			}
		}
		return;
	}
	long coff[NB];
	for (int j = 0; j < NB; j++) coff[j] = (long)(cbase + j * 32 + r32) * a.oc;
	for (int v = 0; v < 16; v++) {
		const int rv = 8 * (v >> 2) + 4 * h + (v & 3), m = mbase + rv;
		const int E = row_e(v, rv);
		// f64 arithmetic on integers below 2^53: (double)(tot - 8 qsum) exactly
		const double q8 = 8.0 * (double)row_q(v, rv); // 0 for int8 weights
		if (m >= a.M) continue;
		int r = m, jj = 0;
		if (a.ni != 1) r = m / a.ni, jj = m - r * a.ni;
		float *orow = a.o + (long)r * a.orr + (long)jj * a.oj;
		for (int j = 0; j < NB; j++) {
			if (cbase + j * 32 + r32 >= w.C) continue;
			orow[coff[j]] = act_out<ACT>(sc[j] * (float)ldexp(totd(j, v) - (PAIRS && (j & 1) ? 0.0 : q8), E - 23));
		}
	}
}

// Wait until at most N vector-memory loads of this wave are outstanding
// (loads complete in order; copies to LDS count as loads).
template <int N>
__device__ inline void wait_vm()
{
	static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit count");
	asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// One 1 KiB global -> LDS copy by a wave: lane l moves the 16 bytes at
// sbase + voff into LDS address lds + 16 l (voff = 16 l). Issued with inline
// assembly so that the compiler, which cannot tell these copies apart from
// the LDS reads of other ring stages, does not drain all outstanding copies
// before every read; the K loop waits for its stage explicitly (wait_vm).
__device__ inline void copy_to_lds(const uint8_t *sbase, unsigned voff, unsigned lds)
{
	asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds) : "memory");
}

// The epilogue of qgemm_k<BITS, 1> (a chain, and the row op when the tile
// holds whole lines): the tile's products go to LDS first (the ring's space,
// free after the K loop), each wave its own 32 x 128 block from its
// accumulators (rows of the reference's loop are left for the second pass),
// lines rowstr(BN) floats apart (odd: one thread per line walks distinct
// banks). Then all 512 threads take the tile line by line, a wave 64
// channels at a time: the reference's loop for special rows, the chain
// (finish), and either the store or, with the row op, the line ops of
// rowop_lds_k (kern_layer.hip) in the reference's order: the sums one
// thread per line in index order, the max, the exponentials, the division
// and the scaling spread over every thread. The chain's code appears once
// (a loop, not unrolled per output), which keeps the kernel small.
constexpr int rowstr(int C) { return C | 1; }
constexpr int EPI_LDS = BM * rowstr(BN) * 4 + BM * 4; // line values and one scalar per line

template <bool PAIRS, bool W8, class TotD>
__device__ void staged_epilogue(const tgk_qgemm_args &a, const tgk_qweight &w, const Scratch &s, int m0, int c0, int wm, int g, int lane,
				int wave, int tid, bool row, float *L, TotD totd)
{
	constexpr int STR = rowstr(BN);
	const int nl = a.M - m0 < BM ? a.M - m0 : BM, cw = w.C - c0 < BN ? w.C - c0 : BN; // the tile's lines and channels
	float *lv = L + BM * STR; // one scalar per line
	wait_vm<0>();
	__syncthreads(); // every wave is past its last read of the ring
	{
		const int mbase = m0 + wm * 32, r32 = lane & 31, h = lane >> 5;
		const TileRows<4> t = tile_rows<4>(a, w, s, mbase, c0 + g * 128, lane);
		if (!__any(t.spr == 2)) { // no split row in the block (the common case): unrolled, each sum from its own register
			__builtin_amdgcn_s_waitcnt(0x0f70); // vmcnt(0): the row data and scales, once
#pragma unroll
			for (int v = 0; v < 16; v++) {
				const int rv = 8 * (v >> 2) + 4 * h + (v & 3);
				const int E = __shfl(t.Er, rv);
				const double q8 = W8 ? 0.0 : 8.0 * (double)__shfl(t.Qr, rv);
#pragma unroll
				for (int j = 0; j < 4; j++) {
					const double tj = W8 || (PAIRS && (j & 1)) ? totd(j, v) : totd(j, v) - q8;
					L[(wm * 32 + rv) * STR + g * 128 + j * 32 + r32] = t.sc[j] * (float)ldexp(tj, E - 23);
				}
			}
		} else
		for (int v = 0; v < 16; v++) {
			const int rv = 8 * (v >> 2) + 4 * h + (v & 3), m = mbase + rv;
			const int E = __shfl(t.Er, rv), sp = __shfl(t.spr, rv);
			const double q8 = 8.0 * (double)__shfl(t.Qr, rv); // 0 for int8 weights
			for (int j = 0; j < 4; j++) {
				const int c = c0 + g * 128 + j * 32 + r32;
				const double gv = ldexp(totd(j, v) - (PAIRS && (j & 1) ? 0.0 : q8), E - 23);
				L[(wm * 32 + rv) * STR + g * 128 + j * 32 + r32] =
					t.sc[j] * (float)(sp == 2 && c < w.C ? gv + outlier_sum(s, w, m, c) : gv); // split rows (m < M: sp is 0 past M)
			}
		}
	}
	// a wave takes lines wave, wave + 8, ... (16 of them), 64 channels at a time
	const int spl = lane < 16 && wave + 8 * lane < nl ? s.special[m0 + wave + 8 * lane] & 1 : 0;
	__syncthreads();
	if (__any(spl)) // lines of the reference's loop: their products, a wave per line
		for (int i = 0; i < 16; i++)
			if (__shfl(spl, i)) {
				const int l = wave + 8 * i;
				float t[BN / 64];
				ref_line<BN / 64>(a, w, m0 + l, c0, lane, t);
				for (int q = 0; q < BN / 64; q++) {
					const int c = (BN / 64) * lane + q;
					if (c < cw) L[l * STR + c] = w.scale[c0 + c] * t[q];
				}
			}
	// the chain, four lines at a time: for each instruction, every operand
	// load of the four lines first, then the arithmetic (the operation chosen
	// once per instruction, not per element); results back to LDS (no global
	// store here, so no load waits for a store)
	for (int i0 = 0; i0 < 16; i0 += 4) {
		float v[16];
		int rr[4], jr[4];
		for (int il = 0; il < 4; il++) {
			const int l = wave + 8 * (i0 + il), m = m0 + (l < nl ? l : 0);
			rr[il] = m / a.ni;
			jr[il] = m - rr[il] * a.ni;
			for (int q = 0; q < 4; q++) {
				const int c = lane + 64 * q;
				v[il * 4 + q] = l < nl && c < cw ? L[l * STR + c] : 0.0f;
			}
		}
		for (int e = 0; e < a.nepi; e++) {
			const int kind = a.epi[e].kind, op = a.epi[e].op;
			if (kind == TGK_EW_UN) {
				switch (op) {
#define EPU(K) \
	case K: \
		for (int u = 0; u < 16; u++) v[u] = tg_uop(K, v[u]); \
		break;
					EPU(TGM_NEG) EPU(TGM_TANH) EPU(TGM_RELU) EPU(TGM_SIGMOID) EPU(TGM_EXP) EPU(TGM_SQRT) EPU(TGM_GELU)
					EPU(TGM_SILU) EPU(TGM_SOFTPLUS) EPU(TGM_LOG) EPU(TGM_SIN) EPU(TGM_COS) EPU(TGM_FLOOR)
					default: EPU(TGM_STEP)
#undef EPU
				}
				continue;
			}
			const int mode = a.epi[e].mode;
			const float *xp = a.epi[e].x;
			const long xr = a.epi[e].xr;
			float x[16];
			for (int il = 0; il < 4; il++) {
				const int l = wave + 8 * (i0 + il);
				const float *p = xp + (long)rr[il] * xr;
				for (int q = 0; q < 4; q++) {
					const int c = lane + 64 * q, cc = c0 + (c < cw ? c : 0);
					x[il * 4 + q] = l >= nl ? 0.0f : mode == 0 ? p[(long)jr[il] * a.oj + (long)cc * a.oc] : mode == 1 ? p[0] : p[cc];
				}
			}
			const bool rev = kind == TGK_EW_BINR;
			switch (op) {
#define EPB(K) \
	case K: \
		for (int u = 0; u < 16; u++) v[u] = rev ? tg_bop(K, x[u], v[u]) : tg_bop(K, v[u], x[u]); \
		break;
				EPB(TGK_ADD) EPB(TGK_SUB) EPB(TGK_MUL) EPB(TGK_DIV) EPB(TGK_MAX)
				default: EPB(TGK_MIN)
#undef EPB
			}
		}
		for (int il = 0; il < 4; il++) {
			const int l = wave + 8 * (i0 + il);
			for (int q = 0; q < 4; q++)
				if (l < nl && lane + 64 * q < cw) L[l * STR + lane + 64 * q] = v[il * 4 + q];
		}
	}
	__syncthreads();
	// row op (whole lines in the tile: c0 = 0, channel stride 1)
	const int C = cw;
	auto line_sum = [&](int l, bool sq) { // in index order from 0.0f
		const float *y = L + l * STR;
		float sum = 0.0f;
		int i = 0;
		for (; i + 8 <= C; i += 8) {
			float z[8];
			for (int u = 0; u < 8; u++) z[u] = y[i + u];
			for (int u = 0; u < 8; u++) sum += sq ? z[u] * z[u] : z[u];
		}
		for (; i < C; i++) sum += sq ? y[i] * y[i] : y[i];
		return sum;
	};
	if (row && a.rowop == TGM_SOFTMAX) {
		if (tid < nl) { // x[0] when it is nan, else the largest of x[0] and the non-nan x[i]
			const float *y = L + tid * STR;
			float mx = -INFINITY;
			for (int i = 1; i < C; i++) mx = fmaxf(mx, y[i]);
			lv[tid] = isnan(y[0]) ? y[0] : fmaxf(y[0], mx);
		}
		__syncthreads();
		for (int l = wave; l < nl; l += 8)
			for (int c = lane; c < C; c += 64) L[l * STR + c] = expf(L[l * STR + c] - lv[l]);
		__syncthreads();
		if (tid < nl) lv[tid] = line_sum(tid, false);
		__syncthreads();
		for (int l = wave; l < nl; l += 8)
			for (int c = lane; c < C; c += 64) L[l * STR + c] = L[l * STR + c] / lv[l];
		__syncthreads();
	} else if (row) {
		if (tid < nl) lv[tid] = 1.0f / sqrtf(line_sum(tid, true) / (float)C + 1e-6f);
		__syncthreads();
		for (int l = wave; l < nl; l += 8)
			for (int c = lane; c < C; c += 64) L[l * STR + c] = L[l * STR + c] * lv[l];
		__syncthreads();
	}
	// the stores, after every load: four channels per lane and store where
	// the line is contiguous and 16-byte aligned
	for (int l = wave; l < nl; l += 8) {
		const int m = m0 + l, r = m / a.ni, jj = m - r * a.ni;
		float *o = a.o + (long)r * a.orr + (long)jj * a.oj + (long)c0 * a.oc;
		const float *y = L + l * STR;
		if (a.oc == 1 && ((size_t)o & 15) == 0) {
			for (int c = 4 * lane; c < cw; c += 256) {
				if (c + 4 <= cw) *(float4 *)(o + c) = make_float4(y[c], y[c + 1], y[c + 2], y[c + 3]);
				else
					for (int u = c; u < cw; u++) o[u] = y[u];
			}
		} else
			for (int c = lane; c < cw; c += 64) o[(long)c * a.oc] = y[c];
	}
}

// Large batches. 512 threads = 8 waves; the workgroup computes a 128 x 256
// tile (rows x channels): wave w (group g = w / 4, rows wm = w % 4) a 32 x 128
// block as four 32 x 32 blocks of v_mfma_i32_32x32x32_i8 for each of the three
// digit planes (192 accumulator registers). Each 64-input step needs 24 KiB of
// digits and 8 (int4) or 16 (int8) KiB of weights, copied straight from global
// memory into a ring of 4 LDS stages (global_load_lds, 1 KiB per wave
// instruction, no registers): group 0 copies the digits, group 1 the weights,
// 3 stages ahead.
//
// The two waves on a SIMD (w and w + 4) belong to different groups and take
// turns: the kernel runs in barrier-separated slots, and in each slot one
// group reads its next step's fragments from LDS (and issues its copies) while
// the other runs the 24 MFMAs of its current step, group 1 one slot behind
// group 0. The matrix cores of every SIMD so always have a wave with operands
// in registers. Per stage kt: group 0 reads it in slot 2 kt, multiplies in
// 2 kt + 1; group 1 reads in 2 kt + 1, multiplies in 2 kt + 2. Stage kt + 3
// is copied in the reading slot of stage kt into the ring slot of stage
// kt - 1, whose last reader (group 1) finished in slot 2 kt - 1; a wave waits
// for its copies of stage kt + 1 at the end of its reading slot of stage kt,
// before the barrier that precedes the first read of stage kt + 1.
//
// EPI 1: the epilogue applies the chain (a.epi), and the row op when `row`
// (the tile holds whole lines: one channel tile, channel stride 1), through
// LDS (staged_epilogue). EPI 2 / 3: the chain is a lone tanh / silu, applied
// as each output is stored (the stores' code then stays as small as without it).

template <int BITS, int EPI = 0>
__global__ __launch_bounds__(512) void qgemm_k(tgk_qgemm_args a, tgk_qweight w, Scratch s, int gx, int gy, int row)
{
	constexpr int S = 4;                          // ring stages (128 or 160 KiB)
	constexpr int AST = 24 * 1024;                // 4 row blocks x 2 substeps x 3 digits x 1 KiB
	constexpr int BST = BITS == 4 ? 8192 : 16384; // 8 channel blocks x 2 substeps x 512 B or 1 KiB
	constexpr int STG = AST + BST;
	constexpr int GA = BITS == 4 ? 4 : 6, GB = 4; // copies per wave per stage: group 0, group 1
	constexpr int LDSB = EPI == 1 && EPI_LDS > S * STG ? (EPI_LDS + 1023) / 1024 * 1024 : S * STG;
	__shared__ __attribute__((aligned(1024))) uint8_t lds[LDSB];
	const int tid = threadIdx.x, lane = tid & 63;
	const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), g = wave >> 2, wm = wave & 3;
	// XCD-aware tile order: workgroups are dealt to the 8 XCDs round robin, so
	// renumber them to give each XCD a contiguous band of row tiles (its L2
	// then holds those rows' digits for every channel tile).
	int id = blockIdx.x, T = gx * gy;
	if (T % 8 == 0) id = (id % 8) * (T / 8) + id / 8;
	const int bm = id / gx, bn = id % gx;
	const int m0 = bm * BM, c0 = bn * BN, nk = w.Kp / KB, kblocks = w.Kp / 32;
	const uint8_t *gA = (const uint8_t *)s.dig + (long)(m0 / 32) * kblocks * 3072;
	const uint8_t *gB = BITS == 4 ? w.wg + (long)(c0 / 64) * kblocks * 1024 : w.w + (long)(c0 / 32) * kblocks * 1024;
	const unsigned voff = lane * 16;
	const unsigned lds0 = (unsigned)(size_t)(__attribute__((address_space(3))) uint8_t *)lds;
	// int4: group 0 wave wm copies digit pieces 0-3 of row block wm, group 1
	// wave wm pieces 4 and 5 and both 32-input halves of channel-block pair wm
	// (4 copies per wave in both groups); int8: group 0 wave wm the six digit
	// pieces of row block wm, group 1 wave wm weight pieces 4 wm .. 4 wm + 3
	// (channel block p / 2, half p % 2). Weight piece p lands at AST + 1 KiB p.
	auto issue = [&](int kt) {
		const unsigned dst = lds0 + (unsigned)((kt % S) * STG);
		const uint8_t *src = gA + (long)wm * kblocks * 3072 + (long)kt * 6144;
		if (BITS == 4) {
			if (g == 0)
				for (int i = 0; i < 4; i++) copy_to_lds(src + i * 1024, voff, dst + (wm * 6 + i) * 1024);
			else {
				for (int i = 4; i < 6; i++) copy_to_lds(src + i * 1024, voff, dst + (wm * 6 + i) * 1024);
				for (int i = 0; i < 2; i++)
					copy_to_lds(gB + (long)wm * kblocks * 1024 + (long)kt * 2048 + i * 1024, voff, dst + AST + (2 * wm + i) * 1024);
			}
		} else if (g == 0) {
			for (int i = 0; i < GA; i++) copy_to_lds(src + i * 1024, voff, dst + (wm * GA + i) * 1024);
		} else {
			for (int i = 0; i < GB; i++) {
				const int p = wm * GB + i;
				copy_to_lds(gB + (long)(p >> 1) * kblocks * 1024 + (p & 1) * 1024 + (long)kt * 2048, voff, dst + AST + p * 1024);
			}
		}
	};
	v16i acc[3][4];
	for (int l = 0; l < 3; l++)
		for (int j = 0; j < 4; j++)
			for (int v = 0; v < 16; v++) acc[l][j][v] = 0;
	// int4: bf[kk][q] holds the raw bytes of channel-block pair 2 g + q, the
	// operand of column blocks 2 q + 1 (S1); blo its low nibbles, the operand
	// of column blocks 2 q (S0), masked one pair ahead
	constexpr int NBF = BITS == 4 ? 2 : 4;
	v4i af[2][3];
	v4i bf[2][NBF];
	v4i blo;
	auto fread = [&](int kt) {
		for (int kk = 0; kk < 2; kk++) {
			const uint8_t *A = lds + (kt % S) * STG + wm * 6144 + kk * 3072 + lane * 16;
			for (int l = 0; l < 3; l++) af[kk][l] = *(const v4i *)(A + l * 1024);
			const uint8_t *B = lds + (kt % S) * STG + AST + g * (BST / 2) + kk * 1024 + lane * 16;
			for (int j = 0; j < NBF; j++) bf[kk][j] = *(const v4i *)(B + j * 2048);
		}
	};
	auto mfma = [&](int l, int j, int kk, const v4i &b) {
		acc[l][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[kk][l], b, acc[l][j], 0, 0, 0);
	};
	auto mm = [&]() {
		if constexpr (BITS == 4) {
			for (int i = 0; i < 4; i++) {
				const int kk = i >> 1, q = i & 1;
				for (int l = 0; l < 3; l++) mfma(l, 2 * q, kk, blo);
				if (i + 1 < 4) blo = bf[(i + 1) >> 1][(i + 1) & 1] & 0x0f0f0f0f;
				for (int l = 0; l < 3; l++) mfma(l, 2 * q + 1, kk, bf[kk][q]);
				__builtin_amdgcn_sched_group_barrier(0x8, 3, 0); // MFMA
				if (i + 1 < 4) __builtin_amdgcn_sched_group_barrier(0x2, 4, 0); // VALU: the next mask
				__builtin_amdgcn_sched_group_barrier(0x8, 3, 0);
			}
		} else
			for (int kk = 0; kk < 2; kk++)
				for (int j = 0; j < 4; j++)
					for (int l = 0; l < 3; l++) mfma(l, j, kk, bf[kk][j]);
	};
	auto bar = [&]() {
		__builtin_amdgcn_sched_barrier(0);
		__builtin_amdgcn_s_barrier();
		__builtin_amdgcn_sched_barrier(0);
		asm volatile("" ::: "memory"); // LDS changed behind the compiler's back: reload it
	};
	for (int st = 0; st < S - 1; st++)
		if (st < nk) issue(st);
	wait_vm<0>();
	bar();
	if (g == 1) bar(); // group 1 runs one slot behind
	for (int kt = 0; kt < nk; kt++) {
		// reading slot
		fread(kt); // the LDS reads first: the copies are issued while they land
		if (kt + S - 1 < nk) issue(kt + S - 1);
		__builtin_amdgcn_s_waitcnt(0xc07f); // lgkmcnt(0): the fragments are in registers
		if (kt + 1 < nk) { // this wave's copies of stage kt + 1 have landed (later stages may be in flight)
			const int later = (kt + S - 1 < nk ? S - 1 : nk - 1 - kt) - 1;
			if (g == 0) {
				if (later <= 0) wait_vm<0>();
				else if (later == 1) wait_vm<GA>();
				else wait_vm<2 * GA>();
			} else {
				if (later <= 0) wait_vm<0>();
				else if (later == 1) wait_vm<GB>();
				else wait_vm<2 * GB>();
			}
		}
		if constexpr (BITS == 4) blo = bf[0][0] & 0x0f0f0f0f; // the first mask here, so the first MFMA waits for nothing
		bar();
		// multiplying slot
		mm();
		bar();
	}
	if (g == 0) bar(); // both groups pass the same number of barriers
	// int4: column block 2 q + 1's sums are (S1 - S0) / 16 (exact), codes without the +8 bias
	auto tot = [&](int j, int v) {
		const long long t = combine(acc[0][j][v], acc[1][j][v], acc[2][j][v]);
		if (BITS == 4 && (j & 1)) return (t - combine(acc[0][j - 1][v], acc[1][j - 1][v], acc[2][j - 1][v])) / 16;
		return t;
	};
	auto totd = [&](int j, int v) {
		const double t = combine_d(acc[0][j][v], acc[1][j][v], acc[2][j][v]);
		if (BITS == 4 && (j & 1)) return (t - combine_d(acc[0][j - 1][v], acc[1][j - 1][v], acc[2][j - 1][v])) * 0.0625;
		return t;
	};
	if constexpr (EPI == 1) {
		staged_epilogue<BITS == 4, BITS == 8>(a, w, s, m0, c0, wm, g, lane, wave, tid, row != 0, (float *)lds, totd);
		return;
	}
	store_tile<4, false, EPI == 2 ? TGM_TANH : EPI == 3 ? TGM_SILU : 0, BITS == 4, BITS == 8>(a, w, s, m0 + wm * 32, c0 + g * 128, lane,
								 tile_rows<4>(a, w, s, m0 + wm * 32, c0 + g * 128, lane), tot, totd);
}

typedef unsigned v2u __attribute__((ext_vector_type(2)));

// a pointer the whole wave shares, in scalar registers (the "s" operands of
// the loads below need it there; the compiler may otherwise keep a uniform
// pointer in vector registers when scalar ones run short)
template <class T>
__device__ inline T *sgpr_ptr(T *p)
{
	const unsigned long long u = (unsigned long long)p;
	const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)u), hi = __builtin_amdgcn_readfirstlane((unsigned)(u >> 32));
	return (T *)(((unsigned long long)hi << 32) | lo);
}

// Register loads of the small-batch kernel, issued with inline assembly: the
// compiler does not track them, so each ring slot is waited for explicitly
// (wait_vm) and then "touched" (an empty asm that reads and writes the slot's
// registers), which keeps every use of the slot below the wait.
__device__ inline void ld16(v4i &d, const void *sbase, unsigned voff)
{
	asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(d) : "v"(voff), "s"(sbase) : "memory");
}
__device__ inline void ld8(v2u &d, const void *sbase, unsigned voff)
{
	asm volatile("global_load_dwordx2 %0, %1, %2" : "=v"(d) : "v"(voff), "s"(sbase) : "memory");
}
__device__ inline void touch(v4i &x) { asm volatile("" : "+v"(x)); }
__device__ inline void touch(v2u &x) { asm volatile("" : "+v"(x)); }

// Small and medium batches. A workgroup of W waves computes a 32 x 32 NB tile
// (rows x channels); wave w sums the 32-input blocks kb = w, w + W, ..., loading
// its fragments straight from global memory into a ring of P register slots
// (no LDS staging: no fragment is shared between the waves), so P blocks are
// in flight per wave. Lanes of rows at or beyond M read row 0's bytes (the
// same addresses as row 0's lanes, served by the same memory requests): a
// one-row batch fetches one row of digits, and those rows' outputs are not
// written. Past a wave's last block the loads repeat the last block (the
// index is clamped) and the slot is not multiplied, so there is no branch
// around a load. The first min(NB, W) waves write the tile's column blocks
// (each wave's share of the epilogue runs beside the others'); every wave
// leaves its partial sums in LDS and each writer adds its blocks' W partial
// sums. Each partial sum and every sum of them is an integer below 2^48 in
// magnitude, so each f64 addition is exact.
template <int BITS, int NB, int W, int P = 4>
__global__ __launch_bounds__(64 * W) void qgemv_k(tgk_qgemm_args a, tgk_qweight w, Scratch s, int gx)
{
	// P ring slots (blocks in flight per wave)
	constexpr int LB = BITS == 4 ? 8 : 16;        // weight bytes per lane per block
	constexpr int NL = 3 + NB;                    // load instructions per block
	static_assert((P - 1) * NL < 64, "the ring's wait count must fit vmcnt");
	typedef typename std::conditional<BITS == 4, v2u, v4i>::type bfrag;
	__shared__ double red[W > 1 ? NB * W * 16 * 64 : 1]; // every wave's sums of every column block
	const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int bx = blockIdx.x % gx, by = blockIdx.x / gx;
	const int m0 = by * 32, c0 = bx * NB * 32, kblocks = w.Kp / 32;
	const int mrem = a.M - m0; // rows of this tile that exist (>= 1)
	const unsigned voffA = (unsigned)(((lane >> 5) * 32 + ((lane & 31) < mrem ? (lane & 31) : 0)) * 16);
	const unsigned voffB = (unsigned)(lane * LB);
	const int8_t *A = s.dig + (long)(m0 / 32) * kblocks * 3072;
	const uint8_t *B = w.w + (long)(c0 / 32) * kblocks * (LB * 64);
	v16i acc[3][NB];
	for (int l = 0; l < 3; l++)
		for (int j = 0; j < NB; j++)
			for (int v = 0; v < 16; v++) acc[l][j][v] = 0;
	v4i af[P][3];
	bfrag bf[P][NB];
	const int n = (kblocks - wave + W - 1) / W; // blocks of this wave
	auto load = [&](int u, int i) {
		long kb = wave + (long)i * W;
		kb = kb < kblocks ? kb : kblocks - 1;
		for (int l = 0; l < 3; l++) ld16(af[u][l], A + (kb * 3 + l) * 1024, voffA);
		for (int j = 0; j < NB; j++) {
			const uint8_t *b = B + ((long)j * kblocks + kb) * (LB * 64);
			if constexpr (BITS == 4) ld8(bf[u][j], b, voffB);
			else ld16(bf[u][j], b, voffB);
		}
	};
	for (int u = 0; u < P; u++) load(u, u);
	// The tile's outputs are written by min(NB, W) waves, NBW column blocks
	// each (wave w blocks w NBW ..). Their row data are fetched now for the
	// narrow tiles (the latency then hides behind the K loop; the wide tiles
	// keep the registers).
	constexpr int NBW = W >= NB ? 1 : NB / W;
	const bool writer = wave < (W >= NB ? NB : W);
	const int jw = wave * NBW;
	constexpr bool PRE = NB <= 2;
	TileRows<NBW> rows;
	if constexpr (PRE) rows = tile_rows<NBW>(a, w, s, m0, c0 + 32 * jw, lane);
	for (int i0 = 0; i0 < n; i0 += P) {
		for (int u = 0; u < P; u++) {
			wait_vm<(P - 1) * NL>(); // slot u's loads are the oldest P - 1 groups back
			for (int l = 0; l < 3; l++) touch(af[u][l]);
			for (int j = 0; j < NB; j++) touch(bf[u][j]);
			if (i0 + u < n) {
				for (int j = 0; j < NB; j++) {
					v4i wv;
					if constexpr (BITS == 4) wv = unpack4(bf[u][j].x, bf[u][j].y);
					else wv = bf[u][j];
					for (int l = 0; l < 3; l++) acc[l][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[u][l], wv, acc[l][j], 0, 0, 0);
				}
			}
			load(u, i0 + u + P);
		}
	}
	wait_vm<0>(); // the ring's last (unused) loads have landed before the wave goes on
	// ... and until then every ring register stays allocated to its load: the
	// compiler sees each slot read here, after the wait, so it cannot hand a
	// register with a load still in flight to another value (an in-flight
	// load would overwrite it)
	for (int u = 0; u < P; u++) {
		for (int l = 0; l < 3; l++) touch(af[u][l]);
		for (int j = 0; j < NB; j++) touch(bf[u][j]);
	}
	if (W > 1) { // slot (column block j, wave u): red[((j W + u) 16 + v) 64 + lane]
		for (int j = 0; j < NB; j++)
			for (int v = 0; v < 16; v++) red[((j * W + wave) * 16 + v) * 64 + lane] = combine_d(acc[0][j][v], acc[1][j][v], acc[2][j][v]);
		__syncthreads();
		if (!writer) return;
	}
	// the block's sum of this wave's column block jw + j (exact, as above)
	auto totd = [&](int j, int v) {
		if constexpr (W > 1) {
			double t = 0.0;
			for (int u = 0; u < W; u++) t += red[(((jw + j) * W + u) * 16 + v) * 64 + lane];
			return t;
		} else
			return combine_d(acc[0][j][v], acc[1][j][v], acc[2][j][v]);
	};
	if constexpr (!PRE) rows = tile_rows<NBW>(a, w, s, m0, c0 + 32 * jw, lane);
	store_tile<NBW, NBW <= 2>(a, w, s, m0, c0 + 32 * jw, lane, rows, [&](int j, int v) { return (long long)totd(j, v); }, totd);
}

// Batches of at most 16 rows: v_mfma_i32_16x16x64_i8 (16 rows x 16 channels
// x 64 inputs per instruction; lane l holds row or channel l % 16 and inputs
// 16 (l / 16) .. +15 of the step, and outputs rows 4 (l / 16) .. +3 of
// channel l % 16). A workgroup of W waves computes one 16-channel tile over
// all K: wave w takes the 64-input steps w, w + W, ... (NS of them), and
// issues every load of its steps (weights straight from global memory, the
// digits of its steps) before its first MFMA, step by step, so a device full
// of workgroups has all of the weight in flight at once (config 2: 256
// workgroups, 8 MiB). The loads are inline assembly, as in qgemv_k: step i is
// waited for with an exact count (the 4 (NS - 1 - i) younger loads may still
// be in flight) and its registers are touched after the wait, so the
// compiler neither drains every load before the first MFMA nor hands an
// in-flight register to another value. Each operand is one contiguous run
// per 16 lanes of the large-batch layouts: the digit layout's row block 0
// (rows past M read row 0's bytes, the same addresses), and 8 (int4) or 16
// (int8) bytes of the 32 x 32 weight fragment holding the lane's channel and
// inputs. Every wave leaves its exact sums (planes combined in f64: integers
// below 2^53) in LDS; wave 0 adds them and writes the 256 outputs through
// epilogue() (special rows take the reference's loop there).
template <int BITS>
using gemv16_frag = typename std::conditional<BITS == 4, v2u, v4i>::type;

template <int BITS, int NS, int I>
__device__ inline void gemv16_steps(v4i (&af)[NS][3], gemv16_frag<BITS> (&bf)[NS], v4i (&acc)[3], int nvalid)
{
	if constexpr (I < NS) {
		wait_vm<4 * (NS - 1 - I)>();
		touch(bf[I]);
		for (int l = 0; l < 3; l++) touch(af[I][l]);
		if (I < nvalid) {
			v4i wv;
			if constexpr (BITS == 4) wv = unpack4(bf[I].x, bf[I].y);
			else wv = bf[I];
			for (int l = 0; l < 3; l++) acc[l] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[I][l], wv, acc[l], 0, 0, 0);
		}
		gemv16_steps<BITS, NS, I + 1>(af, bf, acc, nvalid);
	}
}

template <int BITS, int NS, int W>
__global__ __launch_bounds__(64 * W) void gemv16_k(tgk_qgemm_args a, tgk_qweight w, Scratch s)
{
	static_assert(4 * NS <= 64, "the wait count must fit vmcnt");
	__shared__ double red[W][4][64];
	const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int t = blockIdx.x, r = lane & 15, g = lane >> 4;
	const int nks = w.Kp / 64, kblocks = w.Kp / 32;
	constexpr int LB = BITS == 4 ? 8 : 16; // weight bytes per lane per fragment
	// operand bases (uniform) and the lane's offsets within them
	const int8_t *A = s.dig;
	const uint8_t *B = w.w + (long)(t >> 1) * kblocks * (64 * LB);
	const unsigned offA = (unsigned)((r < a.M ? r : 0) * 16 + (g & 1) * 512 + (g >> 1) * 3072);
	const unsigned offB = (unsigned)((g >> 1) * (64 * LB) + ((g & 1) * 32 + (t & 1) * 16 + r) * LB);
	v4i af[NS][3];
	gemv16_frag<BITS> bf[NS];
	for (int i = 0; i < NS; i++) {
		int st = wave + i * W;
		st = st < nks ? st : nks - 1; // past the wave's last step: reload the last step (not multiplied)
		if constexpr (BITS == 4) ld8(bf[i], B, offB + (unsigned)st * (2 * 64 * LB));
		else ld16(bf[i], B, offB + (unsigned)st * (2 * 64 * LB));
		for (int l = 0; l < 3; l++) ld16(af[i][l], A, offA + (unsigned)st * 6144 + l * 1024);
	}
	v4i acc[3] = { { 0, 0, 0, 0 }, { 0, 0, 0, 0 }, { 0, 0, 0, 0 } };
	gemv16_steps<BITS, NS, 0>(af, bf, acc, (nks - wave + W - 1) / W);
	for (int v = 0; v < 4; v++) red[wave][v][lane] = combine_d(acc[0][v], acc[1][v], acc[2][v]);
	// wave 0's epilogue reads (its rows' exponents, classes and sums of q,
	// its channel's scale), all issued here, before the barrier: read one
	// row at a time between the output stores, each would wait for the
	// previous store (the compiler cannot tell the buffers apart)
	const int c = t * 16 + r;
	int re[4] = { 0, 0, 0, 0 }, rc[4] = { 0, 0, 0, 0 };
	long long rq[4] = { 0, 0, 0, 0 };
	float sc = 0.0f;
	if (wave == 0) {
		for (int v = 0; v < 4; v++) {
			const int m = 4 * g + v < a.M ? 4 * g + v : 0;
			re[v] = s.e[m], rc[v] = s.special[m], rq[v] = s.qsum[m];
		}
		sc = w.scale[c < w.C ? c : w.C - 1];
	}
	__syncthreads();
	if (wave) return;
	for (int v = 0; v < 4; v++) {
		double tot = 0.0;
		for (int u = 0; u < W; u++) tot += red[u][v][lane]; // exact: integers below 2^53
		epilogue_sc(a, w, s, 4 * g + v, c, (long long)tot, re[v], rc[v], rq[v], sc);
	}
}

template <int BITS, int NS, int W>
void launch_gemv16(hipStream_t st, const tgk_qgemm_args *a, Scratch s)
{
	gemv16_k<BITS, NS, W><<<a->w->Cp / 16, 64 * W, 0, st>>>(*a, *a->w, s);
}

// gemv1_k's K loop over its NL weight loads: load i is waited for with the
// NL - 1 - i younger ones still in flight, its registers touched, then used
template <int NL, int I, class F>
__device__ inline void gemv1_steps(v4i (&bf)[NL], F &dots)
{
	if constexpr (I < NL) {
		wait_vm<NL - 1 - I>();
		touch(bf[I]);
		dots(I, bf[I]);
		gemv1_steps<NL, I + 1>(bf, dots);
	}
}

// gemv1_k's row when it is a candidate (FUSED: one row, unit stride): the
// decision of resolve_k, taken by the workgroup from the row in its
// registers (thread tid holds the 16-input groups tid + 256 u), so every
// workgroup reaches the same decision and values as resolve_k would.
// Returns the row's class (0 its grid, 1 the reference's loop, 2 split). For
// a split row, lane j < 16 of wave 0 gets channel 16 t + j's sum before the
// scale in `acc32` (the exact grid sum of the rest in f64 plus the outlier
// terms in increasing input order, rounded once: the epilogue's split
// value), and workgroup 0 leaves the split in the scratch (digits, exponent,
// sum of q, outliers), as resolve_k does, for a product that reuses them.
struct FusedSplitLds {
	TgqHist h;
	long long red[4][16];
	long long qs[4];
	int cnt[4][2];
	unsigned rmax[4];
	int L;
	int ok[TGQ_MAX_OUT];
	float ox[TGQ_MAX_OUT];
};

template <int GX>
__device__ int fused_resolve(const tgk_qweight &w, const Scratch &s, const float (&v)[GX][16], int E, int n, int t, int tid, int lane,
			     int wave, FusedSplitLds &F, float &acc32)
{
	static_assert(GX <= 2, "outlier order below: two groups per thread");
	const int K = w.K;
	if (tid < 64) F.h.cnt[tid] = 0, F.h.bmax[tid] = 0, F.h.mass[tid] = 0;
	__syncthreads();
	for (int u = 0; u < GX; u++)
		if (16 * (tid + 256 * u) < K) (void)tgq_hist16(&F.h, v[u], E);
	__syncthreads();
	if (wave == 0) {
		const int L = tgq_decide(&F.h, n, lane);
		if (lane == 0) F.L = L;
	}
	__syncthreads();
	const int L = F.L;
	if (L <= 0) return L < 0 ? 1 : 0;
	// the outliers, and the largest of the rest
	float rm = 0.0f;
	unsigned om[GX];
	int inc[GX], cnt[GX];
	for (int u = 0; u < GX; u++) {
		om[u] = 0;
		if (16 * (tid + 256 * u) < K)
			for (int i = 0; i < 16; i++) {
				if (tgq_outlier(v[u][i], E, L)) om[u] |= 1u << i;
				else rm = fmaxf(rm, fabsf(v[u][i]));
			}
		cnt[u] = inc[u] = __popc(om[u]);
		for (int d = 1; d < 64; d <<= 1) { // inclusive scan over the wave's lanes
			const int x = __shfl_up(inc[u], d);
			if (lane >= d) inc[u] += x;
		}
	}
	rm = wave_max(rm);
	if (lane == 0) F.rmax[wave] = __float_as_uint(rm); // non-negative: the bits order as the values
	if (lane == 63)
		for (int u = 0; u < GX; u++) F.cnt[wave][u] = inc[u];
	__syncthreads();
	const int Er = tgq_exponent(__uint_as_float(max(max(F.rmax[0], F.rmax[1]), max(F.rmax[2], F.rmax[3]))), 0);
	// the outlier list in increasing input order: groups u, then waves, then lanes
	int tot = 0;
	for (int u = 0; u < GX; u++) {
		int at = tot + inc[u] - cnt[u];
		for (int ww = 0; ww < wave; ww++) at += F.cnt[ww][u];
		for (int ww = 0; ww < 4; ww++) tot += F.cnt[ww][u];
		for (int i = 0; i < 16; i++)
			if ((om[u] >> i) & 1) {
				if (at < TGQ_MAX_OUT) F.ok[at] = 16 * (tid + 256 * u) + i, F.ox[at] = v[u][i];
				at++;
			}
	}
	const int nin = tot < TGQ_MAX_OUT ? tot : TGQ_MAX_OUT; // tot <= J(n) <= TGQ_MAX_OUT (tgq_decide)
	// the rest's grid: exact integer sums for the workgroup's 16 channels, one at a time
	float r[GX][16];
	long long qr = 0, tl = 0;
	int8_t *gblk = tgq_row_base(s.dig, 0, w.Kp);
#pragma unroll
	for (int u = 0; u < GX; u++) {
		const int k0 = 16 * (tid + 256 * u);
#pragma unroll
		for (int i = 0; i < 16; i++) r[u][i] = k0 >= K || ((om[u] >> i) & 1) ? 0.0f : v[u][i];
		if (k0 >= K) continue;
		if (t == 0) qr += tgq_put16(gblk, k0, r[u], Er, false, tl); // the scratch copy (this thread wrote the grid's there)
		else
#pragma unroll
			for (int i = 0; i < 16; i++) qr += (int)rintf(ldexpf(r[u][i], 23 - Er));
	}
#pragma unroll 1
	for (int j = 0; j < 16; j++) {
		const int c = t * 16 + j;
		long long acc = 0;
		if (c < w.C)
#pragma unroll
			for (int u = 0; u < GX; u++) {
				const int k0 = 16 * (tid + 256 * u);
				if (k0 < K)
#pragma unroll
					for (int i = 0; i < 16; i++) {
						const int q = (int)rintf(ldexpf(r[u][i], 23 - Er)); // exact: |q| < 2^23
						if (q) acc += (long long)code_orig(w, c, k0 + i) * q;
					}
			}
		acc = wave_sum(acc);
		if (lane == 0) F.red[wave][j] = acc;
	}
	qr = wave_sum(qr);
	if (lane == 0) F.qs[wave] = qr;
	__syncthreads();
	if (t == 0) {
		const int nout = tgq_nout(w.Kp);
		for (int j = tid; j < nout; j += 256) s.ok[j] = j < nin ? F.ok[j] : -1, s.ox[j] = j < nin ? F.ox[j] : 0.0f;
		if (tid == 0) s.e[0] = Er, s.qsum[0] = F.qs[0] + F.qs[1] + F.qs[2] + F.qs[3], s.special[0] = 2;
	}
	if (wave == 0 && lane < 16 && t * 16 + lane < w.C) {
		const int c = t * 16 + lane;
		const long long g = F.red[0][lane] + F.red[1][lane] + F.red[2][lane] + F.red[3][lane];
		double o = 0.0;
		for (int j = 0; j < nin; j++) o += (double)code_orig(w, c, F.ok[j]) * (double)F.ox[j];
		acc32 = (float)(ldexp((double)g, Er - 23) + o);
	}
	return 2;
}

// One activation row (M = 1) and int4 weights: exact integer dot products by
// 4-way int8 dot instructions (v_dot4_i32_i8), no MFMA padding. A workgroup
// of four waves computes 16 channels (half of a 32-channel fragment block)
// over all K; wave w takes 32-input blocks 4 NL w .. 4 NL w + 4 NL - 1, and
// lane l of a wave reads, from fragment block 4 i + l / 16 of its range,
// the 16 bytes of two adjacent channels (l % 8 pairs) of input half
// (l % 16) / 8: 16-byte loads, each 16 lanes one 128-byte run, NL of them per
// lane issued at once (config 2: 256 workgroups, 8 lanes' worth of 16 bytes
// each, the whole 8 MiB in flight). The row's digits are in LDS,
// [block][digit][half][16 bytes], read by every lane with the same block and
// half (a broadcast).
// FUSED: the workgroup makes those digits itself from the row (unit stride,
// 16-byte aligned, K a multiple of 16): max |x|, exponent, peak test and sum
// of q by block reductions, exactly as the digit kernels do, so no digit
// kernel runs before it; workgroup 0 also writes the digits and row data to
// the scratch (a later product may reuse them). Otherwise the digits come
// from the scratch. The row and digit loads are issued before the weight
// loads and waited for with a count that leaves the weights in flight (loads
// complete in order), all as inline assembly like qgemv_k's.
template <int NL, bool FUSED>
__global__ __launch_bounds__(256) void gemv1_k(tgk_qgemm_args a, tgk_qweight w, Scratch s)
{
	constexpr int GX = 2; // 16-input groups of the row per thread (FUSED: K <= 8192)
	__shared__ __attribute__((aligned(16))) int8_t dl[256 * 96]; // digits: [block][digit][half][16]
	__shared__ int red[4][8][2][3];
	__shared__ unsigned smx[4];
	__shared__ int sbad[4];
	__shared__ long long sq[4], stl[4];
	const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
	const int t = blockIdx.x, f = lane >> 4, h = (lane >> 3) & 1, pr = lane & 7;
	const int kblocks = w.Kp / 32, K = w.K;
	// the row's loads first (inline assembly: counted by the waits below)
	v4i xv[FUSED ? GX * 4 : 1];
	v4i dv[FUSED ? 1 : 6];
	const uint8_t *xb = sgpr_ptr((const uint8_t *)xrow(a, 0));
	if constexpr (FUSED) {
		for (int u = 0; u < GX; u++) {
			const int k0 = 16 * (tid + 256 * u), kk = k0 < K ? k0 : 0; // past the row: its first group (not used)
			for (int i = 0; i < 4; i++) ld16(xv[u * 4 + i], xb, (unsigned)(kk + 4 * i) * 4);
		}
	} else {
		for (int u = 0; u < 6; u++) { // chunk c = (block, digit, half) of row 0 in the fragment layout
			int c = tid + 256 * u;
			c = c < kblocks * 6 ? c : 0;
			ld16(dv[u], s.dig, (unsigned)((c / 6) * 3072 + ((c % 6) >> 1) * 1024 + (c & 1) * 512));
		}
	}
	// the weights: NL 16-byte loads per lane
	const uint8_t *B = sgpr_ptr(w.w + (long)(t >> 1) * kblocks * 512);
	const unsigned offB = (unsigned)((h * 32 + (t & 1) * 16 + 2 * pr) * 8);
	v4i bf[NL];
	for (int i = 0; i < NL; i++) {
		int kb = wave * 4 * NL + 4 * i + f;
		kb = kb < kblocks ? kb : kblocks - 1; // past the end: reload the last block (not used)
		ld16(bf[i], B, offB + (unsigned)kb * 512);
	}
	// the row's digits into LDS (the weights stay in flight)
	wait_vm<NL>();
	int E = 0, sp0 = 0;
	float v[FUSED ? GX : 1][16];
	if constexpr (FUSED) {
		for (int i = 0; i < GX * 4; i++) touch(xv[i]);
		unsigned mb = 0;
		for (int u = 0; u < GX; u++) {
			for (int i = 0; i < 4; i++)
				for (int e = 0; e < 4; e++) v[u][4 * i + e] = __int_as_float(xv[u * 4 + i][e]);
			if (16 * (tid + 256 * u) < K) tgq_scan16(v[u], mb);
		}
		float mx;
		int bad;
		tgq_scan_end(mb, mx, bad);
		mx = wave_max(mx); // a NaN lane reads 0 here; its row is flagged by `bad`
		bad = __any(bad);
		if (lane == 0) smx[wave] = __float_as_uint(mx), sbad[wave] = bad;
		__syncthreads();
		const float amax = fmaxf(fmaxf(__uint_as_float(smx[0]), __uint_as_float(smx[1])),
					 fmaxf(__uint_as_float(smx[2]), __uint_as_float(smx[3])));
		sp0 = tgq_special(sbad[0] | sbad[1] | sbad[2] | sbad[3], amax);
		E = tgq_exponent(amax, sp0);
	} else {
		for (int u = 0; u < 6; u++) {
			touch(dv[u]);
			const int c = tid + 256 * u;
			if (c < kblocks * 6) *(v4i *)(dl + c * 16) = dv[u]; // chunk c = ((block 3 + digit) 2 + half)
		}
	}
	long long qs = 0, tl = 0; // this thread's share of the sum of q and of the peak tally (FUSED)
	if constexpr (FUSED) {
		int8_t *gblk = tgq_row_base(s.dig, 0, w.Kp);
		for (int u = 0; u < GX; u++) {
			const int k0 = 16 * (tid + 256 * u);
			if (k0 >= w.Kp) break;
			unsigned w0[4] = { 0, 0, 0, 0 }, w1[4] = { 0, 0, 0, 0 }, w2[4] = { 0, 0, 0, 0 }; // zero digits: padding, special rows
			long long tl0 = 0; // the peak tally is taken after the dot products, off the critical path
			if (!sp0 && k0 < K) qs += tgq_digits16(v[u], E, w0, w1, w2, tl0);
			int8_t *p = dl + ((k0 >> 5) * 3 * 2 + ((k0 >> 4) & 1)) * 16;
			*(v4i *)p = v4i{ (int)w0[0], (int)w0[1], (int)w0[2], (int)w0[3] };
			*(v4i *)(p + 32) = v4i{ (int)w1[0], (int)w1[1], (int)w1[2], (int)w1[3] };
			*(v4i *)(p + 64) = v4i{ (int)w2[0], (int)w2[1], (int)w2[2], (int)w2[3] };
			if (t == 0) { // the scratch copy, for a product that reuses these digits
				int8_t *g = gblk + (k0 >> 5) * 3072 + ((k0 >> 4) & 1) * 512;
				*(v4i *)g = v4i{ (int)w0[0], (int)w0[1], (int)w0[2], (int)w0[3] };
				*(v4i *)(g + 1024) = v4i{ (int)w1[0], (int)w1[1], (int)w1[2], (int)w1[3] };
				*(v4i *)(g + 2048) = v4i{ (int)w2[0], (int)w2[1], (int)w2[2], (int)w2[3] };
			}
		}
	}
	__syncthreads();
	// this lane's digits of its NL blocks, read before the first weight wait
	// (up to eight loads per lane: beyond that the registers they take make
	// the compiler move in-flight load registers around, which tests/
	// test_asm_ring.py catches; then each step reads its digits from LDS)
	constexpr bool PRE = NL <= 8;
	const int nkb = kblocks - wave * 4 * NL; // blocks of this wave's range that exist
	auto digits_of = [&](int i, v4i (&d3)[3]) {
		const int kbl = 4 * i + f < nkb ? 4 * i + f : 0;
		const int8_t *d = dl + ((wave * 4 * NL + kbl) * 6 + h) * 16;
		for (int l = 0; l < 3; l++) d3[l] = *(const v4i *)(d + 32 * l);
	};
	v4i dg[PRE ? NL : 1][3];
	if constexpr (PRE)
		for (int i = 0; i < NL; i++) digits_of(i, dg[i]);
	// dot products: channels 2 pr, 2 pr + 1 of the tile, digits 0..2
	int acc[2][3] = { { 0, 0, 0 }, { 0, 0, 0 } };
	auto dots = [&](int i, const v4i &b) {
		if (4 * i + f >= nkb) return;
		v4i d3[3];
		if constexpr (PRE)
			for (int l = 0; l < 3; l++) d3[l] = dg[i][l];
		else
			digits_of(i, d3);
		const v4i c0 = unpack4((unsigned)b.x, (unsigned)b.y), c1 = unpack4((unsigned)b.z, (unsigned)b.w);
		for (int e = 0; e < 4; e++)
			for (int l = 0; l < 3; l++) {
				acc[0][l] = __builtin_amdgcn_sdot4(c0[e], d3[l][e], acc[0][l], false);
				acc[1][l] = __builtin_amdgcn_sdot4(c1[e], d3[l][e], acc[1][l], false);
			}
	};
	gemv1_steps<NL, 0>(bf, dots);
	// lanes with the same channel pair: over the input half (lane bit 3) and block (bits 4, 5)
	for (int o = 8; o < 64; o <<= 1)
		for (int j = 0; j < 2; j++)
			for (int l = 0; l < 3; l++) acc[j][l] += __shfl_xor(acc[j][l], o);
	if (lane < 8)
		for (int j = 0; j < 2; j++)
			for (int l = 0; l < 3; l++) red[wave][lane][j][l] = acc[j][l];
	int special;
	long long qsum;
	float acc32 = 0.0f; // a split row's sum (fused_resolve)
	if constexpr (FUSED) { // the row's sum of q and candidate test (needed only from here on)
		__shared__ FusedSplitLds F;
		for (int u = 0; u < GX; u++)
			if (!sp0 && 16 * (tid + 256 * u) < K) tl += tgq_tally16(v[u], E);
		qs = wave_sum(qs);
		tl = wave_sum(tl);
		if (lane == 0) sq[wave] = qs, stl[wave] = tl;
		__syncthreads();
		qsum = sq[0] + sq[1] + sq[2] + sq[3];
		const long long tally = stl[0] + stl[1] + stl[2] + stl[3];
		special = sp0;
		if (!sp0 && tgq_candidate(tally)) // uniform over the workgroup
			special = fused_resolve<GX>(w, s, v, E, (int)(tally >> TGQ_TALLY_SHIFT), t, tid, lane, wave, F, acc32);
		if (t == 0 && tid == 0 && special != 2) s.e[0] = E, s.special[0] = special, s.qsum[0] = qsum;
	} else {
		__syncthreads();
		E = s.e[0], special = s.special[0], qsum = s.qsum[0];
	}
	if (wave || lane >= 16) return;
	if (FUSED && special == 2) {
		const int c = t * 16 + lane;
		if (c < w.C) *out_at(a, 0, 0, c) = w.scale[c] * acc32;
		return;
	}
	int p3[3] = { 0, 0, 0 };
	for (int u = 0; u < 4; u++)
		for (int l = 0; l < 3; l++) p3[l] += red[u][lane >> 1][lane & 1][l];
	epilogue_with(a, w, s, 0, t * 16 + lane, combine(p3[0], p3[1], p3[2]), E, special, qsum);
}

// gemv1_k for a single row of int4 weights: NL 16-byte weight loads per lane,
// 16 NL >= the row's 32-input blocks (at most 256: K <= 8192)
template <bool FUSED>
bool launch_gemv1(hipStream_t st, const tgk_qgemm_args *a, Scratch s)
{
	const tgk_qweight *w = a->w;
	const int kblocks = w->Kp / 32, g = w->Cp / 16;
	if (a->M != 1 || w->bits != 4 || kblocks > 256) return false;
	if (kblocks <= 16) gemv1_k<1, FUSED><<<g, 256, 0, st>>>(*a, *w, s);
	else if (kblocks <= 32) gemv1_k<2, FUSED><<<g, 256, 0, st>>>(*a, *w, s);
	else if (kblocks <= 64) gemv1_k<4, FUSED><<<g, 256, 0, st>>>(*a, *w, s);
	else if (kblocks <= 128) gemv1_k<8, FUSED><<<g, 256, 0, st>>>(*a, *w, s);
	else gemv1_k<16, FUSED><<<g, 256, 0, st>>>(*a, *w, s);
	return true;
}

// gemv16_k's instantiation for K: W waves of NS steps each, W * NS >= Kp / 64.
// No instantiation may spill a register (a spill of a register whose load is
// still in flight stores the wrong bytes; tests/test_asm_ring.py checks):
// sixteen waves leave 128 registers per wave, too few for int8 weights at
// eight steps, so int8 rows longer than 4096 inputs take qgemv_k.
template <int BITS>
bool launch_small(hipStream_t st, const tgk_qgemm_args *a, Scratch s)
{
	const int nks = a->w->Kp / 64;
	if (a->M > 16 || nks > 16 * 8 || (BITS == 8 && nks > 64)) return false;
	if (nks <= 4) launch_gemv16<BITS, 1, 4>(st, a, s);
	else if (nks <= 8) launch_gemv16<BITS, 2, 4>(st, a, s);
	else if (nks <= 16) launch_gemv16<BITS, 2, 8>(st, a, s);
	else if (nks <= 32) launch_gemv16<BITS, 4, 8>(st, a, s);
	else if (nks <= 64) launch_gemv16<BITS, 8, 8>(st, a, s);
	else if constexpr (BITS == 4) launch_gemv16<BITS, 8, 16>(st, a, s);
	return true;
}

template <int BITS, int NB, int W, int P = 4>
void launch_gemv(hipStream_t st, const tgk_qgemm_args *a, Scratch s)
{
	const int gx = a->w->Cp / (32 * NB), gy = (int)round_up(a->M, 32) / 32;
	qgemv_k<BITS, NB, W, P><<<gx * gy, 64 * W, 0, st>>>(*a, *a->w, s, gx);
}

// Products over at most TGK_REFLOOP_K inputs (a selective SSM's dt projection
// has 16) take the reference's sequential loop for every row
// (runtime/tg_rt.h:132-151): at that length it costs about what the exact
// digit path costs per output (16 inputs: 16 multiplies and 16 adds against
// 12 four-way dot products, the planes' combination and a digit kernel before
// the product), and it needs no digits, no row class and no resolve; every
// output is the reference's bit for bit, at every batch size. A thread takes
// NC channels (c = 256 (NC blockIdx.x + q) + thread, q < NC) over the
// workgroup's rows, U at a time: the U rows' inputs are read first (one round
// trip), the channels' codes are kept in registers as floats, each sum runs
// k = 0 .. K - 1 as the reference's does (product rounded, then the add);
// then the scale and, when `chain`, the chain, each instruction applied to the
// U NC values at once as staged_epilogue applies it.
template <int KM, int NC, int U, bool VEC>
__global__ __launch_bounds__(256, KM <= 16 ? 4 : 1) void qtiny_k(tgk_qgemm_args a, tgk_qweight w, int rows_per_block, int chain)
{
	constexpr int NV = U * NC;
	int c[NC], cc[NC];
	float cf[NC][KM], sc[NC];
	for (int q = 0; q < NC; q++) {
		c[q] = 256 * (NC * blockIdx.x + q) + threadIdx.x;
		cc[q] = c[q] < w.C ? c[q] : w.C - 1;
		for (int k = 0; k < KM; k++) cf[q][k] = k < w.K ? (float)code_orig(w, cc[q], k) : 0.0f;
		sc[q] = w.scale[cc[q]];
	}
	const int m0 = blockIdx.y * rows_per_block, m1 = a.M - m0 < rows_per_block ? a.M : m0 + rows_per_block;
	// row m is batch row r, inner row j (m = r ni + j): the block's first row
	// divided once, then stepped (uniform, no division per row)
	const int r0 = a.ni == 1 ? m0 : m0 / a.ni, j0 = m0 - r0 * a.ni;
	int rb = r0, jb = j0; // row mb's
	for (int mb = m0; mb < m1; mb += U) {
		int rr[U], jr[U];
		float xv[U][KM];
		for (int u = 0; u < U; u++) {
			int r = rb, j = jb + u;
			while (j >= a.ni) j -= a.ni, r++;
			if (mb + u >= m1) r = r0, j = j0; // past the block's rows: a row of it, not stored
			rr[u] = r;
			jr[u] = j;
			const float *x = a.x + (long)r * a.xr + (long)j * a.xj;
			if constexpr (VEC) { // unit stride, 16-byte aligned, K a multiple of 4
				for (int k = 0; k < KM; k += 4) {
					const float4 f = k < w.K ? *(const float4 *)(x + k) : float4{ 0.0f, 0.0f, 0.0f, 0.0f };
					xv[u][k] = f.x, xv[u][k + 1] = f.y, xv[u][k + 2] = f.z, xv[u][k + 3] = f.w;
				}
			} else {
				for (int k = 0; k < KM; k++) xv[u][k] = k < w.K ? x[(long)k * a.xk] : 0.0f;
			}
		}
		// the reference's loop over the K inputs; the padding past K adds
		// 0 x 0 = +0, which leaves every sum as it is (a sum that starts at +0
		// is never -0), so it needs no test
		float v[NV]; // value (u, q) at u NC + q
		for (int u = 0; u < U; u++)
			for (int q = 0; q < NC; q++) {
				float t = 0.0f;
				for (int k = 0; k < KM; k++) t += cf[q][k] * xv[u][k];
				v[u * NC + q] = sc[q] * t;
			}
		for (int e = 0; chain && e < a.nepi; e++) {
			const int kind = a.epi[e].kind, op = a.epi[e].op;
			if (kind == TGK_EW_UN) {
				switch (op) {
#define EPU(K) \
	case K: \
		for (int i = 0; i < NV; i++) v[i] = tg_uop(K, v[i]); \
		break;
					EPU(TGM_NEG) EPU(TGM_TANH) EPU(TGM_RELU) EPU(TGM_SIGMOID) EPU(TGM_EXP) EPU(TGM_SQRT) EPU(TGM_GELU)
					EPU(TGM_SILU) EPU(TGM_SOFTPLUS) EPU(TGM_LOG) EPU(TGM_SIN) EPU(TGM_COS) EPU(TGM_FLOOR)
					default: EPU(TGM_STEP)
#undef EPU
				}
				continue;
			}
			const int mode = a.epi[e].mode;
			float x[NV];
			for (int u = 0; u < U; u++) {
				const float *p = a.epi[e].x + (long)rr[u] * a.epi[e].xr;
				for (int q = 0; q < NC; q++)
					x[u * NC + q] = mode == 0 ? p[(long)jr[u] * a.oj + (long)cc[q] * a.oc] : mode == 1 ? p[0] : p[cc[q]];
			}
			const bool rev = kind == TGK_EW_BINR;
			switch (op) {
#define EPB(K) \
	case K: \
		for (int i = 0; i < NV; i++) v[i] = rev ? tg_bop(K, x[i], v[i]) : tg_bop(K, v[i], x[i]); \
		break;
				EPB(TGK_ADD) EPB(TGK_SUB) EPB(TGK_MUL) EPB(TGK_DIV) EPB(TGK_MAX)
				default: EPB(TGK_MIN)
#undef EPB
			}
		}
		for (int u = 0; u < U; u++)
			if (mb + u < m1)
				for (int q = 0; q < NC; q++)
					if (c[q] < w.C) *out_at(a, rr[u], jr[u], c[q]) = v[u * NC + q];
		jb += U;
		while (jb >= a.ni) jb -= a.ni, rb++;
	}
}

template <int KM, int U>
void launch_qtiny(hipStream_t st, const tgk_qgemm_args *a, int chain)
{
	const tgk_qweight *w = a->w;
	const int rpb = a->M >= 65536 ? 64 : a->M >= 4096 ? 16 : 4;
	const dim3 grid((unsigned)((w->C + 511) / 512), (unsigned)((a->M + rpb - 1) / rpb));
	const bool vec = a->xk == 1 && ((size_t)a->x & 15) == 0 && (a->xr & 3) == 0 && (a->ni == 1 || (a->xj & 3) == 0) && (w->K & 3) == 0;
	if (vec) qtiny_k<KM, 2, U, true><<<grid, 256, 0, st>>>(*a, *w, rpb, chain);
	else qtiny_k<KM, 2, U, false><<<grid, 256, 0, st>>>(*a, *w, rpb, chain);
}

template <int BITS>
int launch_gemm(hipStream_t st, const tgk_qgemm_args *a, Scratch s, int Mp)
{
	const tgk_qweight *w = a->w;
	if (w->K <= TGK_REFLOOP_K) { // the reference's loop for every row (no digits were made)
		const int chain = a->nseg <= 1; // a chain over segmented outputs is the caller's (tgk_qgemm_chain)
		if (w->K <= 16) launch_qtiny<16, 4>(st, a, chain);
		else launch_qtiny<32, 2>(st, a, chain);
		return chain ? TGK_DID_CHAIN : 0;
	}
	const int gx = w->Cp / BN, gy = Mp / BM;
	const long rt = round_up(a->M, 32) / 32, cb = w->Cp / 32;
	if ((long)gx * gy >= 128 && rt > 2) { // enough 128 x 256 tiles for the LDS kernel
		if (a->nepi == 1 && a->epi[0].kind == TGK_EW_UN && (a->epi[0].op == TGM_TANH || a->epi[0].op == TGM_SILU) && !a->rowop &&
		    a->nseg <= 1) { // a lone tanh or silu: inline in the stores
			if (a->epi[0].op == TGM_TANH) qgemm_k<BITS, 2><<<gx * gy, 512, 0, st>>>(*a, *w, s, gx, gy, 0);
			else qgemm_k<BITS, 3><<<gx * gy, 512, 0, st>>>(*a, *w, s, gx, gy, 0);
			return TGK_DID_CHAIN;
		}
		const int row = a->rowop && gx == 1 && a->oc == 1;
		if ((a->nepi || row) && a->nseg <= 1) { // the chain in the epilogue, and the row op when a tile holds whole lines
			qgemm_k<BITS, 1><<<gx * gy, 512, 0, st>>>(*a, *w, s, gx, gy, row);
			return TGK_DID_CHAIN | (row ? TGK_DID_ROWOP : 0);
		}
		qgemm_k<BITS><<<gx * gy, 512, 0, st>>>(*a, *w, s, gx, gy, 0);
		return 0;
	}
	if (BITS == 4 && launch_gemv1<false>(st, a, s)) return 0; // one row
	if (launch_small<BITS>(st, a, s)) return 0;               // at most 16 rows
	// up to 64 rows, or too few tiles: 32 x (32 NB) tiles, NB as large as
	// still fills the device; W waves split K, about 16 32-input blocks each
	// for the wider tiles and 8-32 for one-block-wide ones (measured: at one
	// block wide, four waves beat eight at K = 4096 and two at K = 1024)
	const int kb = w->Kp / 32;
	if (rt * cb / 4 >= 256) {
		if (kb >= 128) launch_gemv<BITS, 4, 4>(st, a, s);
		else if (kb >= 64) launch_gemv<BITS, 4, 2>(st, a, s);
		else launch_gemv<BITS, 4, 1>(st, a, s);
	} else if (rt * cb / 2 >= 256) {
		if (kb >= 128) launch_gemv<BITS, 2, 4>(st, a, s);
		else if (kb >= 64) launch_gemv<BITS, 2, 2>(st, a, s);
		else launch_gemv<BITS, 2, 1>(st, a, s);
	} else {
		if (kb >= 256) launch_gemv<BITS, 1, 8>(st, a, s);
		else if (kb >= 32) launch_gemv<BITS, 1, 4>(st, a, s);
		else if (kb >= 16) launch_gemv<BITS, 1, 2>(st, a, s);
		else launch_gemv<BITS, 1, 1>(st, a, s);
	}
	return 0;
}

// The repacking of tgk_qweight_pack done on the device, from codes already in
// device memory: one thread per packed byte (and per padded scale), every
// byte of the packed area written (padding: code 0).
__global__ __launch_bounds__(256) void qweight_pack_k(uint8_t *pw, float *ps, uint8_t *pg, const uint8_t *codes, const float *scale,
						      int bits, int axis, int C, int K, int Kp, int Cp)
{
	const long kblocks = Kp / 32, lb = bits == 8 ? 16 : 8, nb = (long)Cp * Kp * bits / 8, ng = bits == 4 ? nb : 0;
	tgk_qweight w{};
	w.orig = (uint8_t *)codes, w.bits = bits, w.axis = axis, w.C = C, w.K = K;
	auto code = [&](int c, int k) { return c < C && k < K ? code_orig(w, c, k) : 0; };
	for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < nb + Cp + ng; i += (long)gridDim.x * blockDim.x) {
		if (i >= nb + Cp) { // int4: the large-batch kernel's copy (channel-block pairs)
			const long j = i - nb - Cp, frag = j / 1024, pr = frag / kblocks, kb = frag - pr * kblocks;
			const int lane = (int)((j / 16) & 63), b = (int)(j % 16);
			const int c = (int)(pr * 64 + (lane & 31)), k = (int)(kb * 32 + (lane >> 5) * 16 + b);
			pg[j] = (uint8_t)(((unsigned)(code(c, k) + 8) & 15u) | (((unsigned)code(c + 32, k) & 15u) << 4));
			continue;
		}
		if (i >= nb) { // the scales, padded with zeros to Cp
			const int c = (int)(i - nb);
			ps[c] = c < C ? scale[c] : 0.0f;
			continue;
		}
		const long frag = i / (64 * lb), cb = frag / kblocks, kb = frag - cb * kblocks;
		const int lane = (int)((i / lb) & 63), b = (int)(i % lb);
		const int c = (int)(cb * 32 + (lane & 31)), k0 = (int)(kb * 32 + (lane >> 5) * 16);
		if (bits == 8) pw[i] = (uint8_t)(int8_t)code(c, k0 + b);
		else pw[i] = (uint8_t)((unsigned)(code(c, k0 + b) + 8) | ((unsigned)(code(c, k0 + b + 8) + 8) << 4));
	}
}

} // namespace

size_t tgk_qweight_dev_bytes(int bits, int C, int K)
{
	const long Kp = round_up(K, KB), Cp = round_up(C, BN), nb = round_up(Cp * Kp * bits / 8, 256);
	return (size_t)nb + (size_t)round_up(Cp * 4, 256) + (bits == 4 ? (size_t)nb : 0);
}

int tgk_qweight_pack_dev(tgk_qweight *w, void *dst, const uint8_t *codes, const float *scale, int bits, int axis, int C, int K,
			 hipStream_t st)
{
	memset(w, 0, sizeof *w);
	w->C = C, w->K = K, w->bits = bits, w->axis = axis;
	w->Kp = (int)round_up(K, KB);
	w->Cp = (int)round_up(C, BN);
	const long nb = (long)w->Cp * w->Kp * bits / 8;
	w->w = (uint8_t *)dst;
	w->scale = (float *)((uint8_t *)dst + round_up(nb, 256));
	w->wg = bits == 4 ? (uint8_t *)dst + round_up(nb, 256) + round_up((long)w->Cp * 4, 256) : nullptr;
	w->orig = (uint8_t *)codes;
	const long n = nb + w->Cp + (bits == 4 ? nb : 0);
	const long blocks = (n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096;
	qweight_pack_k<<<(unsigned)blocks, 256, 0, st>>>(w->w, w->scale, w->wg, codes, scale, bits, axis, C, K, w->Kp, w->Cp);
	return hipGetLastError() == hipSuccess ? 0 : -1;
}

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
	uint8_t *hg = bits == 4 ? (uint8_t *)malloc(nb) : nullptr; /* the large-batch kernel's copy */
	if (bits == 4 && !hg) {
		free(h);
		free(hs);
		return -1;
	}
	if (bits == 4) memset(h, 0x88, nb), memset(hg, 0x08, nb); /* padding codes 0 */
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
				uint8_t *g = hg + (((size_t)(c >> 6) * kblocks + (k >> 5)) * 64 + lane) * 16 + kb;
				*g = c & 32 ? (uint8_t)((*g & 0x0f) | (((unsigned)code & 15u) << 4)) : (uint8_t)((*g & 0xf0) | t);
			}
		}
		hs[c] = scale[c];
	}
	int rc = 0;
	if (hipMalloc(&w->w, nb) != hipSuccess || hipMalloc(&w->scale, (size_t)w->Cp * sizeof(float)) != hipSuccess ||
	    hipMalloc(&w->orig, ob) != hipSuccess || (bits == 4 && hipMalloc(&w->wg, nb) != hipSuccess))
		rc = -1;
	if (!rc && bits == 4 && hipMemcpyAsync(w->wg, hg, nb, hipMemcpyHostToDevice, st) != hipSuccess) rc = -1;
	if (!rc && (hipMemcpyAsync(w->w, h, nb, hipMemcpyHostToDevice, st) != hipSuccess ||
		    hipMemcpyAsync(w->scale, hs, (size_t)w->Cp * sizeof(float), hipMemcpyHostToDevice, st) != hipSuccess ||
		    hipMemcpyAsync(w->orig, codes, ob, hipMemcpyHostToDevice, st) != hipSuccess || hipStreamSynchronize(st) != hipSuccess))
		rc = -1;
	free(h);
	free(hs);
	free(hg);
	return rc;
}

int tgk_qweight_pack_i8(tgk_qweight *w, const int8_t *codes, const float *scale, int bits, int C, int K, hipStream_t st)
{
	if (bits == 8) return tgk_qweight_pack(w, (const uint8_t *)codes, scale, 8, 0, C, K, st);
	const size_t n = (size_t)C * K; /* int4: two codes per byte, element i in byte i / 2, low nibble first */
	uint8_t *q = (uint8_t *)calloc((n + 1) / 2, 1);
	if (!q) return -1;
	for (size_t i = 0; i < n; i++) q[i >> 1] |= (uint8_t)(((unsigned)codes[i] & 15u) << ((i & 1) * 4));
	const int rc = tgk_qweight_pack(w, q, scale, 4, 0, C, K, st);
	free(q);
	return rc;
}

void tgk_qweight_free(tgk_qweight *w)
{
	if (w->w) (void)hipFree(w->w);
	if (w->wg) (void)hipFree(w->wg);
	if (w->scale) (void)hipFree(w->scale);
	if (w->orig) (void)hipFree(w->orig);
	memset(w, 0, sizeof *w);
}

size_t tgk_qgemm_scratch(int M, int Kp)
{
	long Mp = round_up(M, BM);
	return (size_t)Mp * Kp * 3 + (size_t)Mp * (sizeof(long long) + 2 * sizeof(int) + tgq_nout(Kp) * (sizeof(int) + sizeof(float))) + 256;
}

tgk_qdig tgk_qgemm_digit_area(void *scratch, int M, int Kp)
{
	const Scratch s = carve(scratch, (int)round_up(M, BM), Kp);
	return tgk_qdig{ s.dig, s.qsum, s.e, s.special, s.ok, s.ox };
}

void tgk_qgemm_digits(hipStream_t st, const tgk_qgemm_args *a, void *scratch)
{
	const tgk_qweight *w = a->w;
	if (!w || !w->w || !a->x || !scratch || a->M <= 0 || a->ni <= 0 || w->K <= 0) return; /* nothing valid to launch */
	if (w->K <= TGK_REFLOOP_K) return;                                                   /* the product takes the reference's loop */
	int Mp = (int)round_up(a->M, BM);
	const Scratch s = carve(scratch, Mp, w->Kp);
	const int nkb = w->Kp / 32, M = a->M, K = w->K;
	if (M >= 512 && nkb <= 128) { // 16 rows per block
		const bool vec = a->xk == 1 && ((size_t)a->x & 15) == 0 && (a->xr & 3) == 0 && (a->ni == 1 || (a->xj & 3) == 0) &&
				 (K & 15) == 0;
		// 16 waves; 8 for many rows of at most 2048 inputs: then two blocks fit
		// on a CU (registers), one loading while the other computes and stores
		// (measured: K = 2048, 65536 rows: 178 us against 235 with one 32-row
		// block of 16 waves per CU, at a streaming read-then-write floor of 173)
		const int WM = M >= 8192 && nkb <= 64 ? 8 : 16;
		// at least 4 waves (for short rows some only resolve candidates); the
		// first min(W, 8) resolve, one histogram each
		const int W = nkb / 2 < WM ? ((nkb + 1) / 2 < 4 ? 4 : (nkb + 1) / 2) : WM, nb = (M + 15) / 16, pairs = (nkb + 1) / 2;
		// very large batches: the candidates the coarse test leaves are
		// resolved after the digits by a pass of their own at full occupancy
		// (tgk_qgemm_split), not by the first RW waves of each block while the
		// others wait (the same decisions either way; measured on config 5's
		// gated rows, 2 M lines of 512 inputs: 1.8 + 1.5 ms against 3.9; on
		// 65,536 lines the extra launch cost more than it saved)
		const bool defer = M >= DEFER_RESOLVE_ROWS;
		const int RW = defer ? 0 : W < 8 ? W : 8;
		const size_t lds = (size_t)RW * sizeof(TgqHist);
		if (pairs <= W) {
			if (vec) digits_tile16_k<1, true><<<nb, W * 64, lds, st>>>(*a, s, K, w->Kp, M, RW);
			else digits_tile16_k<1, false><<<nb, W * 64, lds, st>>>(*a, s, K, w->Kp, M, RW);
		} else if (pairs <= 2 * W) {
			if (vec) digits_tile16_k<2, true><<<nb, W * 64, lds, st>>>(*a, s, K, w->Kp, M, RW);
			else digits_tile16_k<2, false><<<nb, W * 64, lds, st>>>(*a, s, K, w->Kp, M, RW);
		} else {
			if (vec) digits_tile16_k<4, true><<<nb, W * 64, lds, st>>>(*a, s, K, w->Kp, M, RW);
			else digits_tile16_k<4, false><<<nb, W * 64, lds, st>>>(*a, s, K, w->Kp, M, RW);
		}
		if (defer) tgk_qgemm_split(st, a, scratch);
	} else if (M < 512 && w->Kp >= 2048 && w->Kp <= 16384) { // few long rows: a block per row
		const bool vec = a->xk == 1 && ((size_t)a->x & 15) == 0 && (a->xr & 3) == 0 && (a->ni == 1 || (a->xj & 3) == 0) &&
				 (K & 15) == 0;
		const int G = (w->Kp / 16 + 255) / 256;
		if (G <= 1) {
			if (vec) digits_row_k<1, true><<<M, 256, 0, st>>>(*a, s, K, w->Kp, M);
			else digits_row_k<1, false><<<M, 256, 0, st>>>(*a, s, K, w->Kp, M);
		} else if (G <= 2) {
			if (vec) digits_row_k<2, true><<<M, 256, 0, st>>>(*a, s, K, w->Kp, M);
			else digits_row_k<2, false><<<M, 256, 0, st>>>(*a, s, K, w->Kp, M);
		} else {
			if (vec) digits_row_k<4, true><<<M, 256, 0, st>>>(*a, s, K, w->Kp, M);
			else digits_row_k<4, false><<<M, 256, 0, st>>>(*a, s, K, w->Kp, M);
		}
	} else if (w->Kp <= 1024)
		digits_k<1><<<(M + 3) / 4, 256, 0, st>>>(*a, s, K, w->Kp, M);
	else
		digits_k<4><<<(M + 3) / 4, 256, 0, st>>>(*a, s, K, w->Kp, M);
}

void tgk_qgemm_split(hipStream_t st, const tgk_qgemm_args *a, void *scratch)
{
	const tgk_qweight *w = a->w;
	const int M = a->M;
	if (!w || !a->x || !scratch || M <= 0 || a->ni <= 0 || w->K <= TGK_REFLOOP_K) return;
	const Scratch s = carve(scratch, (int)round_up(M, BM), w->Kp);
	const long blocks = (M + 3) / 4;
	const unsigned nb = (unsigned)(blocks < 16384 ? blocks : 16384);
	const bool vec = a->xk == 1 && ((size_t)a->x & 15) == 0 && (a->xr & 3) == 0 && (a->ni == 1 || (a->xj & 3) == 0) && (w->K & 15) == 0;
	if (vec) resolve_k<true><<<nb, 256, 0, st>>>(*a, s, w->K, w->Kp, M);
	else resolve_k<false><<<nb, 256, 0, st>>>(*a, s, w->K, w->Kp, M);
}

int tgk_qgemm_mfma(hipStream_t st, const tgk_qgemm_args *a, void *scratch)
{
	const tgk_qweight *w = a->w;
	if (!w || !w->w || !w->scale || (w->bits == 4 && !w->wg) || !a->x || !a->o || !scratch || a->M <= 0 || a->ni <= 0) return 0;
	int Mp = (int)round_up(a->M, BM);
	Scratch s = carve(scratch, Mp, w->Kp);
	return w->bits == 8 ? launch_gemm<8>(st, a, s, Mp) : launch_gemm<4>(st, a, s, Mp);
}

namespace {

// The chain over a product's output in place, for the kernels that write
// the products alone: one thread per output
__global__ __launch_bounds__(256) void chain_k(tgk_qgemm_args a, int C, long total)
{
	const long t = (long)blockIdx.x * 256 + threadIdx.x;
	if (t >= total) return;
	const int m = (int)(t / C), c = (int)(t - (long)m * C), r = m / a.ni, jj = m - r * a.ni;
	float *o = a.o + (long)r * a.orr + (long)jj * a.oj + (long)c * a.oc;
	*o = finish(a, r, jj, c, *o);
}

} // namespace

void tgk_qgemm_chain(hipStream_t st, const tgk_qgemm_args *a)
{
	const long total = (long)a->M * a->w->C;
	if (a->nepi <= 0 || total <= 0) return;
	chain_k<<<(unsigned)((total + 255) / 256), 256, 0, st>>>(*a, a->w->C, total);
}

bool tgk_qgemm_fusable(const tgk_qgemm_args *a)
{
	const tgk_qweight *w = a->w;
	return w && w->w && a->x && a->M == 1 && w->bits == 4 && w->K > TGK_REFLOOP_K && w->Kp <= 8192 && a->xk == 1 &&
	       ((size_t)a->x & 15) == 0 && (w->K & 15) == 0;
}

int tgk_qgemm_fused(hipStream_t st, const tgk_qgemm_args *a, void *scratch)
{
	const tgk_qweight *w = a->w;
	if (!w || !w->w || !w->scale || (w->bits == 4 && !w->wg) || !a->x || !a->o || !scratch || a->M <= 0 || a->ni <= 0) return 0;
	if (!tgk_qgemm_fusable(a)) {
		tgk_qgemm_digits(st, a, scratch);
		return tgk_qgemm_mfma(st, a, scratch);
	}
	const int Mp = (int)round_up(a->M, BM);
	launch_gemv1<true>(st, a, carve(scratch, Mp, w->Kp));
	return 0;
}

int tgk_qgemm(hipStream_t st, const tgk_qgemm_args *a, void *scratch)
{
	if (tgk_qgemm_fusable(a)) return tgk_qgemm_fused(st, a, scratch);
	tgk_qgemm_digits(st, a, scratch);
	return tgk_qgemm_mfma(st, a, scratch);
}
