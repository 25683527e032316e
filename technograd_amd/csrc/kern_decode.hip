// Kernels of the KV-cache decoder (tg_decode.cpp) for models in the Qwen3
// importer's layout (examples/qwen3/import.py). Each computes the values the
// fixed-length graph computes, with the same f32 operations in the same
// order (this file is compiled with -ffp-contract=off), so a decoded token's
// logits equal the fixed-length forward's at that position bit for bit.
#include "tg_kern.h"
#include "tg_devmath.h"
#include "tg_qdigits.h"

#include <math.h>

namespace {

// RoPE on the normed, scaled q and k lines of a chunk of token rows (row =
// s * T0 + i at position p0 + i): v = x * cos[p] + (x @ Rot) * sin[p], as the
// graph's `x * cosT + (x @ Rot) * sinT`. q lines go to qr [rows][NQ][HD], k
// lines to the K cache; the chunk's v vectors (columns after q and k of the
// projection output) go to the V cache.
__global__ void rope_cache_k(tgk_dec_rope_args a, long total)
{
	const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
	if (t >= total) return;
	const int NL = a.NQ + 2 * a.NKV; // lines per token row: q, k, v
	const long row = t / ((long)NL * a.HD);
	const int rem = (int)(t - row * NL * a.HD), line = rem / a.HD, d = rem - line * a.HD;
	const int s = (int)(row / a.T0), p = a.p0 + (int)(row - (long)s * a.T0);
	float *kv_s = (float *)0;
	if (line >= a.NQ) kv_s = (line < a.NQ + a.NKV ? a.K : a.V) + (long)s * a.kv_seq + a.kv_layer;
	if (line < a.NQ + a.NKV) {
		const long i = (row * (a.NQ + a.NKV) + line) * a.HD + d;
		const float x = a.hq[i], r = a.rt[i];
		const float c = a.cosT[(long)p * a.HD + d], sn = a.sinT[(long)p * a.HD + d];
		const float v = x * c + r * sn;
		if (line < a.NQ) a.qr[(row * a.NQ + line) * a.HD + d] = v;
		else kv_s[((long)(line - a.NQ) * a.P + p) * a.HD + d] = v;
	} else {
		const int j = line - a.NQ - a.NKV;
		kv_s[((long)j * a.P + p) * a.HD + d] = a.qkv[row * a.ctot + (long)(a.NQ + a.NKV) * a.HD + (long)j * a.HD + d];
	}
}

// The same values four at a time: block y takes token rows y, y + gridDim.y,
// ..., a thread four consecutive d of one line (HD % 4 == 0, every operand
// 16-byte aligned: the launcher checks), so a row's sequence and position
// come from one 32-bit division, not two 64-bit ones per element.
__global__ __launch_bounds__(256) void rope_cache4_k(tgk_dec_rope_args a, int rows)
{
	const int NL = a.NQ + 2 * a.NKV, HD4 = a.HD / 4;
	const int e = blockIdx.x * 256 + threadIdx.x; // (line, quad) of a token row
	if (e >= NL * HD4) return;
	const int line = e / HD4, d = (e - line * HD4) * 4;
	auto rot = [](float x, float c, float r, float sn) { return x * c + r * sn; };
	for (int row = blockIdx.y; row < rows; row += gridDim.y) {
		const int s = row / a.T0, p = a.p0 + (row - s * a.T0);
		float *kv_s = nullptr;
		if (line >= a.NQ) kv_s = (line < a.NQ + a.NKV ? a.K : a.V) + (long)s * a.kv_seq + a.kv_layer;
		if (line < a.NQ + a.NKV) {
			const long i = ((long)row * (a.NQ + a.NKV) + line) * a.HD + d;
			const float4 x = *(const float4 *)(a.hq + i), r = *(const float4 *)(a.rt + i);
			const float4 c = *(const float4 *)(a.cosT + (long)p * a.HD + d), sn = *(const float4 *)(a.sinT + (long)p * a.HD + d);
			const float4 v = make_float4(rot(x.x, c.x, r.x, sn.x), rot(x.y, c.y, r.y, sn.y), rot(x.z, c.z, r.z, sn.z),
						     rot(x.w, c.w, r.w, sn.w));
			if (line < a.NQ) *(float4 *)(a.qr + ((long)row * a.NQ + line) * a.HD + d) = v;
			else *(float4 *)(kv_s + ((long)(line - a.NQ) * a.P + p) * a.HD + d) = v;
		} else {
			const int j = line - a.NQ - a.NKV;
			*(float4 *)(kv_s + ((long)j * a.P + p) * a.HD + d) =
				*(const float4 *)(a.qkv + (long)row * a.ctot + (long)(a.NQ + a.NKV) * a.HD + (long)j * a.HD + d);
		}
	}
}

// One decode step's attention: one block per (sequence, KV head) for the GRP
// query heads sharing it, keys at positions 0 .. p. Per query head and key:
// score = sum_d q[d] k[d] in order from 0.0f, times the scale, plus the mask's
// 0; softmax with the reference's max rule, expf, a sequential sum and a
// division; out[d] = sum over keys of prob * v[d] in key order. The
// fixed-length graph's row for this position has further keys whose masked
// scores give probabilities of exactly 0: they change neither the max nor the
// sums. K, then V, stream through LDS in chunks of ck keys: every thread
// loads its share of the next chunk (16-byte loads) before the current one is
// used, so a chunk's loads are in flight while the previous chunk's chains
// run. Each score, each sum and each output stays one thread's sum in order:
// a (key, head) thread per score, a (head, d) thread per output, carried
// across chunks. LDS rows are HD + 4 floats apart: 16-byte reads of
// consecutive rows by consecutive lanes hit distinct banks. HD % 16 == 0.
constexpr int ATT_TPB = 512, ATT_R = 4; // threads; float4 loads per thread and chunk

int attn_chunk(int HD) // keys per chunk: ATT_R float4 loads per thread, at most 64
{
	int ck = 64;
	while (ck > 1 && ck * (HD / 4) > ATT_R * ATT_TPB) ck >>= 1;
	return ck;
}

template <int GRP>
__global__ __launch_bounds__(ATT_TPB) void dec_attn_k(tgk_dec_attn_args a, int ck)
{
	extern __shared__ float4 sh4[];
	const int n = a.p + 1, HD = a.HD, H4 = HD / 4, KS = H4 + 1, nst = (n + 3) & ~3, per = ck * H4;
	float4 *kv = sh4;                  // [ck][KS] the staged chunk of K or V
	float *q = (float *)(kv + ck * KS); // [GRP][HD]
	float *sc = q + GRP * HD;           // [GRP][nst] scores, then probabilities
	float *lv = sc + GRP * nst;         // [GRP] max, then sum
	const int tid = threadIdx.x, s = blockIdx.x / a.NKV, j = blockIdx.x - s * a.NKV;
	const float *K = a.K + (long)s * a.kv_seq + a.kv_layer + (long)j * a.P * HD;
	const float *V = a.V + (long)s * a.kv_seq + a.kv_layer + (long)j * a.P * HD;
	float4 rg[ATT_R];
	auto fetch = [&](const float *base, int c0) { // chunk of keys c0 .. c0 + ck - 1 into registers
		for (int u = 0; u < ATT_R; u++) {
			const int e = tid + u * ATT_TPB, key = c0 + e / H4;
			rg[u] = e < per && key < n ? ((const float4 *)(base + (long)key * HD))[e % H4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
		}
	};
	auto stash = [&]() {
		for (int u = 0; u < ATT_R; u++) {
			const int e = tid + u * ATT_TPB;
			if (e < per) kv[(e / H4) * KS + e % H4] = rg[u];
		}
	};
	for (int e = tid; e < GRP * HD; e += ATT_TPB) q[e] = a.qr[((long)s * a.NQ + j * GRP) * HD + e];
	fetch(K, 0);
	for (int c0 = 0; c0 < n; c0 += ck) {
		__syncthreads(); // the previous chunk's chains are done with kv
		stash();
		__syncthreads();
		fetch(c0 + ck < n ? K : V, c0 + ck < n ? c0 + ck : 0); // next chunk (or V's first) in flight meanwhile
		for (int it = tid; it < ck * GRP; it += ATT_TPB) {
			const int g = it / ck, kk = it - g * ck;
			if (c0 + kk >= n) continue;
			const float4 *kr = kv + kk * KS, *qg = (const float4 *)(q + g * HD);
			float acc = 0.0f;
			for (int d4 = 0; d4 < H4; d4++) {
				const float4 k4 = kr[d4], q4 = qg[d4];
				acc = acc + q4.x * k4.x;
				acc = acc + q4.y * k4.y;
				acc = acc + q4.z * k4.z;
				acc = acc + q4.w * k4.w;
			}
			sc[g * nst + c0 + kk] = acc * a.scale + 0.0f;
		}
	}
	__syncthreads(); // the score chains are done with kv
	stash();         // V's first chunk (fetched during the last K chunk) into kv,
	if (ck < n) fetch(V, ck); // and its second in flight, both during the softmax
	const int wave = tid >> 6, lane = tid & 63;
	for (int g = wave; g < GRP; g += ATT_TPB >> 6) { // max: a wave per query head
		const float *r = sc + g * nst;
		float m = -INFINITY;
		for (int key = 1 + lane; key < n; key += 64) m = fmaxf(m, r[key]);
		for (int w = 32; w > 0; w >>= 1) m = fmaxf(m, __shfl_xor(m, w));
		if (lane == 0) lv[g] = isnan(r[0]) ? r[0] : fmaxf(r[0], m);
	}
	__syncthreads();
	for (int e = tid; e < GRP * nst; e += ATT_TPB) {
		const int g = e / nst;
		if (e - g * nst < n) sc[e] = expf(sc[e] - lv[g]);
	}
	__syncthreads();
	if (tid < GRP) lv[tid] = tg_ordered_sum_pp<6>(sc + tid * nst, n);
	__syncthreads();
	for (int e = tid; e < GRP * nst; e += ATT_TPB) {
		const int g = e / nst;
		if (e - g * nst < n) sc[e] = sc[e] / lv[g];
	}
	constexpr int OI = (GRP * 256 + ATT_TPB - 1) / ATT_TPB; // outputs per thread (HD <= 256)
	float acc[OI];
	for (int u = 0; u < OI; u++) acc[u] = 0.0f;
	for (int c0 = 0; c0 < n; c0 += ck) {
		__syncthreads(); // probabilities final; the previous chunk's chains are done with kv
		if (c0 > 0) {    // (the first chunk is in kv already)
			stash();
			__syncthreads();
			if (c0 + ck < n) fetch(V, c0 + ck);
		}
		const int m = min(ck, n - c0);
		const float *vb = (const float *)kv;
		for (int u = 0; u < OI; u++) {
			const int it = tid + u * ATT_TPB;
			if (it >= GRP * HD) break;
			const int g = it / HD, d = it - g * HD;
			const float *r = sc + g * nst + c0;
			float x = acc[u];
			for (int kk = 0; kk < m; kk++) x = x + r[kk] * vb[kk * (HD + 4) + d];
			acc[u] = x;
		}
	}
	for (int u = 0; u < OI; u++) {
		const int it = tid + u * ATT_TPB;
		if (it >= GRP * HD) break;
		const int g = it / HD, d = it - g * HD;
		a.att[((long)s * a.NQ + j * GRP + g) * HD + d] = acc[u];
	}
}

// The per-head output projections of a decode step, all heads in one launch:
// out[g][t][c] = x_{t,g} @ W_g[:, c] for query head g, token t, x_{t,g} the
// head's attention output [HD]. Each value is the one the digit kernel and
// the matrix-core GEMM produce for that row: the row's exponent E from its
// max |x| (bumped when the top digit would overflow), q_k = rint(x_k 2^(23-E))
// exactly, split into the same three balanced int8 digits, the exact integer
// sum_k code_k q_k = s0 + 256 s1 + 65536 s2 (s_i = sum_k code_k digit_i,k by
// 4-way int8 dot products), scaled by 2^(E-23) in f64, rounded once to f32
// and multiplied by the channel scale; rows with inf, nan or an entry above
// 2^100 take the reference's sequential f32 loop, and candidate rows
// (tg_qdigits.h) are resolved here as the GEMM path resolves them: a wave
// per row, the same decision; a split row's rest gets digits of its own
// grid and its outliers' terms (f64, increasing k) are added to its grid
// sum before the one rounding. One block per (head, 64 columns): the rows'
// digits and the head's code tile sit in LDS; a wave handles 4 rows at a
// time, a lane one column.
// codes: int32 [NQ][HD/4][D], 4 consecutive k's int8 codes per word (k = 4
// k4 + i in byte i); scales [NQ][D]; HD a multiple of 4, att 16-byte aligned.
constexpr int WO_TPB = 512, WO_NW = WO_TPB / 64;
constexpr int wo_nout(int HD) { return HD / 16 < 1 ? 1 : HD / 16 > TGQ_MAX_OUT ? TGQ_MAX_OUT : HD / 16; } // >= J(n), n <= HD
__global__ __launch_bounds__(WO_TPB) void dec_wo_k(const float *att, const int *codes, const float *scales, float *out, int rows, int NQ,
						   int HD, int D)
{
	extern __shared__ int4 dg[]; // [rows][HD/4] digit words {d0, d1, d2, 0} of 4 k's
	const int H4 = HD / 4, n = rows * H4, NO = wo_nout(HD);
	TgqHist *hist = (TgqHist *)(dg + (long)rows * H4); // one per wave
	long long *tq = (long long *)(hist + WO_NW);      // per row: the candidate tally
	float *ox = (float *)(tq + rows);                 // per row: a split row's outliers [NO], values
	int *ok = (int *)(ox + (long)rows * NO);          // and inputs, -1 past the last
	int *Es = ok + (long)rows * NO, *sp = Es + rows, *ct = sp + rows; // ct: [HD/4][64] code words
	const int ctiles = (D + 63) / 64, g = blockIdx.x / ctiles, c0 = (blockIdx.x - g * ctiles) * 64;
	const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
	constexpr int U = 4;
	auto xat = [&](int e) { // the 4 inputs of item e = (row t, k4)
		const int t = e / H4;
		return *(const float4 *)(att + ((long)t * NQ + g) * HD + 4 * (e - t * H4));
	};
	// rows' max |x| (as bits: non-negative floats order as their bits) and flags
	unsigned *mxb = (unsigned *)Es;
	for (int t = tid; t < rows; t += WO_TPB) mxb[t] = 0, sp[t] = 0, tq[t] = 0;
	for (int e = tid; e < H4 * 64; e += WO_TPB) {
		const int k4 = e >> 6, c = e & 63;
		ct[e] = c0 + c < D ? codes[((long)g * H4 + k4) * D + c0 + c] : 0;
	}
	__syncthreads();
	for (int b = tid; b < n; b += U * WO_TPB) {
		float4 u[U];
		for (int j = 0; j < U; j++) u[j] = xat(min(b + j * WO_TPB, n - 1));
		for (int j = 0; j < U; j++) {
			const int e = b + j * WO_TPB;
			if (e >= n) continue;
			const float4 v = u[j];
			const int bad = !isfinite(v.x) || !isfinite(v.y) || !isfinite(v.z) || !isfinite(v.w);
			const float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))); // a nan never wins fmaxf
			atomicMax(&mxb[e / H4], __float_as_uint(m));
			if (bad) atomicOr(&sp[e / H4], 1);
		}
	}
	__syncthreads();
	for (int t = tid; t < rows; t += WO_TPB) {
		const float mx = __uint_as_float(mxb[t]);
		const int special = tgq_special(sp[t], mx);
		Es[t] = tgq_exponent(mx, special), sp[t] = special;
	}
	__syncthreads();
	// the four inputs' digit words on the grid of E; their tally into *tl
	auto digit_words = [&](const float (&xv)[4], int E, long long *tl) {
		unsigned w0 = 0, w1 = 0, w2 = 0;
		int aq = 0, nx = 0;
		for (int i = 0; i < 4; i++) {
			const float sv = ldexpf(xv[i], 23 - E), rq = rintf(sv);
			const int q = (int)rq; // exact: |q| < 2^23
			aq += abs(q);
			nx += rq != sv;
			int d0, d1, d2;
			tgq_split3(q, d0, d1, d2);
			w0 |= (unsigned)(d0 & 255) << (8 * i);
			w1 |= (unsigned)(d1 & 255) << (8 * i);
			w2 |= (unsigned)(d2 & 255) << (8 * i);
		}
		if (tl && (aq || nx)) atomicAdd((unsigned long long *)tl, (unsigned long long)aq + ((unsigned long long)nx << TGQ_TALLY_SHIFT));
		return make_int4((int)w0, (int)w1, (int)w2, 0);
	};
	for (int b = tid; b < n; b += U * WO_TPB) {
		float4 u[U];
		for (int j = 0; j < U; j++) u[j] = xat(min(b + j * WO_TPB, n - 1));
		for (int j = 0; j < U; j++) {
			const int e = b + j * WO_TPB;
			if (e >= n) continue;
			const int t = e / H4;
			const float xv[4] = { u[j].x, u[j].y, u[j].z, u[j].w };
			dg[e] = sp[t] ? make_int4(0, 0, 0, 0) : digit_words(xv, Es[t], &tq[t]);
		}
	}
	__syncthreads();
	for (int t = tid; t < rows; t += WO_TPB)
		if (!sp[t] && tgq_candidate(tq[t])) sp[t] = 3; // a candidate, resolved below
	__syncthreads();
	// candidates: a wave per row, the GEMM path's resolve (kern_qgemm.hip: resolve_k)
	for (int t = wave; t < rows; t += WO_NW) {
		if (sp[t] != 3) continue; // the same word for the whole wave
		const float *x = att + ((long)t * NQ + g) * HD;
		const int E0 = Es[t];
		auto ld = [&](int gi, float *v) {
			for (int i = 0; i < 16; i++) v[i] = 16 * gi + i < HD ? x[16 * gi + i] : 0.0f;
		};
		TgqCoarse co{}; // the coarse test first (tg_qdigits.h)
		for (int gi = lane; gi < (HD + 15) / 16; gi += 64) {
			float v[16];
			ld(gi, v);
			tgq_coarse16(co, v, E0);
		}
		if (tgq_coarse_grid(tgq_coarse_wave_sum(co), tq[t])) {
			if (lane == 0) sp[t] = 0;
			continue;
		}
		const int L = tgq_resolve(&hist[wave], ld, (HD + 15) / 16, E0, lane);
		if (L <= 0) {
			if (lane == 0) sp[t] = L < 0 ? 1 : 0;
			continue;
		}
		float rm = 0.0f;
		for (int k = lane; k < HD; k += 64)
			if (!tgq_outlier(x[k], E0, L)) rm = fmaxf(rm, fabsf(x[k]));
		for (int o = 32; o > 0; o >>= 1) rm = fmaxf(rm, __shfl_xor(rm, o));
		const int Er = tgq_exponent(rm, 0);
		int nin = 0;
		for (int k40 = 0; k40 < H4; k40 += 64) { // the rest's digits, the outliers in input order
			const int k4 = k40 + lane;
			float xv[4] = { 0.0f, 0.0f, 0.0f, 0.0f };
			unsigned om = 0;
			if (k4 < H4)
				for (int i = 0; i < 4; i++) {
					const float xi = x[4 * k4 + i];
					if (tgq_outlier(xi, E0, L)) om |= 1u << i;
					else xv[i] = xi;
				}
			if (k4 < H4) dg[(long)t * H4 + k4] = digit_words(xv, Er, nullptr);
			const int cnt = __popc(om);
			int inc = cnt;
			for (int d = 1; d < 64; d <<= 1) {
				const int y = __shfl_up(inc, d);
				if (lane >= d) inc += y;
			}
			int at = nin + inc - cnt;
			for (int i = 0; i < 4; i++)
				if ((om >> i) & 1) {
					if (at < NO) ok[(long)t * NO + at] = 4 * k4 + i, ox[(long)t * NO + at] = x[4 * k4 + i];
					at++;
				}
			nin += __shfl(inc, 63);
		}
		for (int j = nin + lane; j < NO; j += 64) ok[(long)t * NO + j] = -1;
		if (lane == 0) Es[t] = Er, sp[t] = 2;
	}
	__syncthreads();
	const int c = lane;
	if (c0 + c >= D) return;
	const float sc = scales[(long)g * D + c0 + c];
	for (int t0 = 4 * wave; t0 < rows; t0 += 4 * WO_NW) {
		int s[4][3] = {};
		int tr[4];
		for (int r = 0; r < 4; r++) tr[r] = min(t0 + r, rows - 1); // rows past the end repeat the last (not stored)
		for (int k4 = 0; k4 < H4; k4++) {
			const int w = ct[k4 * 64 + c];
			for (int r = 0; r < 4; r++) {
				const int4 d = dg[(long)tr[r] * H4 + k4];
				s[r][0] = __builtin_amdgcn_sdot4(w, d.x, s[r][0], false);
				s[r][1] = __builtin_amdgcn_sdot4(w, d.y, s[r][1], false);
				s[r][2] = __builtin_amdgcn_sdot4(w, d.z, s[r][2], false);
			}
		}
		for (int r = 0; r < 4 && t0 + r < rows; r++) {
			const int t = t0 + r;
			auto code = [&](int k) { return (float)(int8_t)(ct[(k >> 2) * 64 + c] >> (8 * (k & 3))); };
			float v;
			if (sp[t] == 1) { // the reference's loop (runtime/tg_rt.h:143-151)
				const float *x = att + ((long)t * NQ + g) * HD;
				float acc = 0.0f;
				for (int k = 0; k < HD; k++) acc += code(k) * x[k];
				v = acc;
			} else { // every term and partial sum an integer below 2^48: exact in f64
				const double tot = (double)s[r][0] + (double)s[r][1] * 256.0 + (double)s[r][2] * 65536.0;
				double o = 0.0; // a split row's outlier terms, in input order
				if (sp[t] == 2)
					for (int j = 0; j < NO && ok[(long)t * NO + j] >= 0; j++) o += (double)code(ok[(long)t * NO + j]) * (double)ox[(long)t * NO + j];
				v = (float)(ldexp(tot, Es[t] - 23) + o);
			}
			out[((long)g * rows + t) * D + c0 + c] = sc * v;
		}
	}
}

// Block-wide reductions (blockDim a multiple of 64, at most 1024); red is
// LDS scratch of 16 entries. Every thread gets the result.
__device__ inline float blk_max(float v, float *red)
{
	for (int w = 32; w > 0; w >>= 1) v = fmaxf(v, __shfl_xor(v, w));
	__syncthreads();
	if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
	__syncthreads();
	float m = red[0];
	for (int i = 1; i < (int)(blockDim.x >> 6); i++) m = fmaxf(m, red[i]);
	return m;
}

// N sums over the block (red: [N][16] in LDS), for thread 0 only
template <int N>
__device__ inline void blk_sums0(unsigned long long (&v)[N], unsigned long long *red)
{
	for (int w = 32; w > 0; w >>= 1)
		for (int i = 0; i < N; i++) v[i] += __shfl_xor(v[i], w);
	__syncthreads();
	if ((threadIdx.x & 63) == 0)
		for (int i = 0; i < N; i++) red[i * 16 + (threadIdx.x >> 6)] = v[i];
	__syncthreads();
	if (threadIdx.x == 0)
		for (int i = 0; i < N; i++) {
			unsigned long long t = 0;
			for (int u = 0; u < (int)(blockDim.x >> 6); u++) t += red[i * 16 + u];
			v[i] = t;
		}
}

// digits of row m of K inputs, values z[0 .. Kp) in LDS (zero from K on), from
// this thread's share of max |z| and of the non-finite flag. The coarse
// histogram (tg_qdigits.h) is kept in the same pass and summed with the sum
// of q and the tally in one block reduction (the rows here are mostly gated
// activations: candidates that the coarse test settles).
__device__ inline void blk_digits(const float *z, int K, int Kp, float mx, int bad, const tgk_qdig &q, int m, float *redf,
				  unsigned long long *redl)
{
	const float amax = blk_max(mx, redf); // nan never wins fmaxf; such rows are flagged by bad
	const int anybad = __syncthreads_or(bad);
	const int special = tgq_special(anybad, amax), E = tgq_exponent(amax, special);
	int8_t *blk = tgq_row_base(q.dig, m, Kp);
	long long qs = 0, tl = 0;
	TgqCoarse co{};
	for (int j = threadIdx.x; j < Kp / 16; j += blockDim.x) {
		float v[16];
		for (int u = 0; u < 16; u++) v[u] = z[16 * j + u];
		qs += tgq_put16(blk, 16 * j, v, E, special, tl);
		if (!special) tgq_coarse16(co, v, E);
	}
	unsigned long long sums[5] = { (unsigned long long)qs, (unsigned long long)tl, co.cnt, co.s0, co.s1 };
	blk_sums0(sums, redl);
	__shared__ int scls;
	if (threadIdx.x == 0) {
		qs = (long long)sums[0], tl = (long long)sums[1];
		co = TgqCoarse{ sums[2], sums[3], sums[4] };
		int cls = special ? TGQ_REF : tgq_candidate(tl) ? TGQ_CAND : TGQ_GRID;
		if (cls == TGQ_CAND && tgq_coarse_grid(co, tl)) cls = TGQ_GRID;
		q.e[m] = E, q.special[m] = cls, q.qsum[m] = qs;
		scls = cls;
	}
	__syncthreads();
	if (scls == TGQ_CAND && threadIdx.x < 64) { // a candidate the coarse test leaves: wave 0 resolves it (the row is in z)
		__shared__ TgqHist hist;
		const int nout = tgq_nout(Kp);
		auto ld = [&](int g, float *v) {
			for (int i = 0; i < 16; i++) v[i] = z[16 * g + i];
		};
		tgq_resolve_row(&hist, ld, K, Kp, E, blk, &q.qsum[m], &q.e[m], &q.special[m], q.ok + (long)m * nout, q.ox + (long)m * nout, nout,
				(int)threadIdx.x);
	}
}

// tgk_dec_norm: one block per token row, NORM_TPB threads, each with at most
// NORM_EPT elements (D <= NORM_TPB * NORM_EPT) whose loads are all issued
// first. The row's sum of squares is the reference's sequential loop over the
// squares (computed in parallel), the scale 1 / sqrtf(sum / D + 1e-6) as the
// row-op kernel, then (h * inv) * g.
constexpr int NORM_TPB = 1024, NORM_EPT = 4;
static_assert(NORM_TPB * NORM_EPT == TGK_DEC_NORM_MAX, "tgk_dec_norm row size");
__global__ __launch_bounds__(NORM_TPB) void dec_norm_k(tgk_dec_norm_args a)
{
	extern __shared__ float4 zs4[]; // [Kp] values, [Kp] squares (16-byte aligned)
	float *zs = (float *)zs4;
	__shared__ float redf[16], inv_s;
	__shared__ unsigned long long redl[5 * 16];
	const int t = blockIdx.x, D = a.D, Kp = a.Kp, tid = threadIdx.x;
	float *z = zs, *sq = zs + Kp, *hr = a.h + (long)t * a.hs;
	float v[NORM_EPT], g[NORM_EPT];
	for (int u = 0; u < NORM_EPT; u++) {
		const int i = tid + u * NORM_TPB, ic = i < D ? i : D - 1;
		v[u] = hr[ic];
		g[u] = a.g[ic];
	}
	if (a.mode == 1) {
		float b[NORM_EPT];
		for (int u = 0; u < NORM_EPT; u++) {
			const int i = tid + u * NORM_TPB;
			b[u] = a.add[(long)t * a.adds + (i < D ? i : D - 1)];
		}
		for (int u = 0; u < NORM_EPT; u++) v[u] = v[u] + b[u];
	} else if (a.mode == 2) { // v + ((o_0 + o_1) + ... + o_{nh-1}), 16 heads' loads at a time
		for (int u = 0; u < NORM_EPT; u++) {
			const int i = tid + u * NORM_TPB;
			if (u > 0 && i >= D) break;
			const float *o = a.o + (long)t * D + (i < D ? i : D - 1);
			float acc = o[0];
			for (int k0 = 1; k0 < a.nh; k0 += 16) {
				float b[16];
				for (int k = 0; k < 16; k++) b[k] = o[(long)(k0 + k < a.nh ? k0 + k : 0) * a.ohead];
				for (int k = 0; k < 16 && k0 + k < a.nh; k++) acc = acc + b[k];
			}
			v[u] = v[u] + acc;
		}
	}
	for (int u = 0; u < NORM_EPT; u++) {
		const int i = tid + u * NORM_TPB;
		if (i >= Kp) break;
		if (i >= D) v[u] = 0.0f;
		else if (a.mode) hr[i] = v[u];
		z[i] = v[u];
		sq[i] = v[u] * v[u];
	}
	__syncthreads();
	if (tid == 0) inv_s = 1.0f / sqrtf(tg_ordered_sum<8>(sq, D) / (float)D + 1e-6f);
	__syncthreads();
	const float inv = inv_s;
	float mx = 0.0f;
	int bad = 0;
	for (int u = 0; u < NORM_EPT; u++) {
		const int i = tid + u * NORM_TPB;
		if (i >= D) break;
		const float nv = v[u] * inv * g[u];
		a.out[(long)t * a.outs + i] = nv;
		z[i] = nv;
		bad |= !isfinite(nv);
		mx = fmaxf(mx, fabsf(nv));
	}
	__syncthreads();
	blk_digits(z, D, Kp, mx, bad, a.q, t, redf, redl);
}

// tgk_dec_hnorm: one wave per head line (4 per block, no block barrier:
// lines past the end leave at once). Same operations as tgk_dec_norm.
__global__ __launch_bounds__(256) void dec_hnorm_k(tgk_dec_hnorm_args a)
{
	extern __shared__ float4 hs4[]; // per wave: [Kp] values, [Kp] squares (16-byte aligned)
	float *hs = (float *)hs4;
	const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, L = blockIdx.x * 4 + w, HD = a.HD, Kp = a.Kp;
	if (L >= a.rows * a.NH) return;
	const int t = L / a.NH, j = L - t * a.NH;
	float *z = hs + (long)w * 2 * Kp, *sq = z + Kp;
	const float *x = a.x + (long)t * a.xs + (long)j * HD;
	for (int i = lane; i < Kp; i += 64) {
		const float v = i < HD ? x[i] : 0.0f;
		z[i] = v;
		sq[i] = v * v;
	}
	__builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
	__builtin_amdgcn_wave_barrier();
	__builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
	float inv = 0.0f;
	if (lane == 0) inv = 1.0f / sqrtf(tg_ordered_sum<8>(sq, HD) / (float)HD + 1e-6f);
	inv = __shfl(inv, 0);
	float mx = 0.0f;
	int bad = 0;
	for (int i = lane; i < HD; i += 64) {
		const float nv = z[i] * inv * a.g[(long)j * HD + i];
		a.out[(long)L * HD + i] = nv;
		z[i] = nv;
		bad |= !isfinite(nv);
		mx = fmaxf(mx, fabsf(nv));
	}
	__builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
	__builtin_amdgcn_wave_barrier();
	__builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
	for (int o = 32; o > 0; o >>= 1) {
		mx = fmaxf(mx, __shfl_xor(mx, o));
		bad |= __shfl_xor(bad, o);
	}
	const int special = tgq_special(bad, mx), E = tgq_exponent(mx, special);
	int8_t *blk = tgq_row_base(a.q.dig, L, Kp);
	long long qs = 0, tl = 0;
	for (int g = lane; g < Kp / 16; g += 64) {
		float v[16];
		for (int u = 0; u < 16; u++) v[u] = z[16 * g + u];
		qs += tgq_put16(blk, 16 * g, v, E, special, tl);
	}
	for (int o = 32; o > 0; o >>= 1) qs += __shfl_xor(qs, o), tl += __shfl_xor(tl, o);
	int cls = special ? TGQ_REF : tgq_candidate(tl) ? TGQ_CAND : TGQ_GRID;
	if (cls == TGQ_CAND) { // (uniform over the wave) the coarse test before any resolve
		TgqCoarse co{};
		for (int g = lane; g < Kp / 16; g += 64) {
			float v[16];
			for (int u = 0; u < 16; u++) v[u] = z[16 * g + u];
			tgq_coarse16(co, v, E);
		}
		if (tgq_coarse_grid(tgq_coarse_wave_sum(co), tl)) cls = TGQ_GRID;
	}
	if (lane == 0) a.q.e[L] = E, a.q.special[L] = cls, a.q.qsum[L] = qs;
	if (cls == TGQ_CAND) { // the wave resolves its line (in z)
		__shared__ TgqHist hist[4];
		const int nout = tgq_nout(Kp);
		auto ld = [&](int g, float *v) {
			for (int i = 0; i < 16; i++) v[i] = z[16 * g + i];
		};
		tgq_resolve_row(&hist[threadIdx.x >> 6], ld, HD, Kp, E, blk, &a.q.qsum[L], &a.q.e[L], &a.q.special[L], a.q.ok + L * nout,
				a.q.ox + L * nout, nout, lane);
	}
}

// Many lines at once (a prompt's token rows, or its head lines): a block of
// NL_TPB threads holds R = NL_E / Kp whole lines, NL_EPT elements per thread
// (all loaded before any is used), and the lines' R sequential sums of squares
// run side by side, one thread each. Line L = t npr + j reads h + t hs + j D
// (updated in place by modes 1 and 2, which need npr == 1), takes gain
// g + j gs, writes out + L D and the digits of row L. The values are the
// same as tgk_dec_norm's and tgk_dec_hnorm's: (h * inv) * g with
// inv = 1 / sqrtf(sum / D + 1e-6), sum the ordered sum of the squares.
struct NormLines {
	float *h;
	long hs;
	int mode;
	const float *add;
	long adds;
	const float *o;
	long ohead;
	int nh;
	const float *g;
	long gs;
	float *out;
	int D, Kp, npr;
	long lines;
	tgk_qdig q;
	int kshift; // Kp = 1 << kshift
};
constexpr int NL_TPB = 256, NL_EPT = 16, NL_E = NL_TPB * NL_EPT;

// LDS: R lines of Kp + 4 floats (16-byte aligned, consecutive lines 4 banks
// apart), then per line its offsets, 1 / rms, exponent and flag
size_t norm_lines_lds(int Kp) { return (size_t)(NL_E / Kp) * ((Kp + 4) * 4 + 8 + 4 * 4); }

__global__ __launch_bounds__(NL_TPB) void norm_lines_k(NormLines a)
{
	extern __shared__ float4 sh4[];
	const int Kp = a.Kp, D = a.D, ks = a.kshift, km = Kp - 1, R = NL_E >> ks, ZS = Kp + 4, tid = threadIdx.x;
	float *z = (float *)sh4; // [R][ZS]: the squares, then the normalized values (0 from D on)
	long *lh = (long *)(z + R * ZS); // line l's offset in h (t hs + j D)
	int *lg = (int *)(lh + R), *lE = lg + R, *lsp = lE + R;
	float *linv = (float *)(lsp + R);
	const long L0 = (long)blockIdx.x * R;
	if (tid < R) { // per line, once (lines past the end repeat the last)
		const long L = L0 + tid < a.lines ? L0 + tid : a.lines - 1;
		const long t = L / a.npr, j = L - t * a.npr;
		lh[tid] = t * a.hs + j * D;
		lg[tid] = (int)(j * a.gs);
	}
	__syncthreads();
	// element u of this thread: e = tid + u NL_TPB, line e >> ks, column e & km
	float v[NL_EPT];
	for (int u = 0; u < NL_EPT; u++) {
		const int e = tid + u * NL_TPB, l = e >> ks, i = e & km;
		v[u] = a.h[lh[l] + (i < D ? i : D - 1)];
	}
	if (a.mode == 1) { // npr == 1: line l is token row L0 + l
		float b[NL_EPT];
		for (int u = 0; u < NL_EPT; u++) {
			const int e = tid + u * NL_TPB, l = e >> ks, i = e & km;
			const long L = L0 + l < a.lines ? L0 + l : a.lines - 1;
			b[u] = a.add[L * a.adds + (i < D ? i : D - 1)];
		}
		for (int u = 0; u < NL_EPT; u++) v[u] = v[u] + b[u];
	} else if (a.mode == 2) { // v + ((o_0 + o_1) + ... + o_{nh-1})
		for (int u = 0; u < NL_EPT; u++) {
			const int e = tid + u * NL_TPB, l = e >> ks, i = e & km;
			const long L = L0 + l < a.lines ? L0 + l : a.lines - 1;
			const float *o = a.o + L * D + (i < D ? i : D - 1);
			float acc = o[0];
			for (int k0 = 1; k0 < a.nh; k0 += 16) {
				float b[16];
				for (int k = 0; k < 16; k++) b[k] = o[(long)(k0 + k < a.nh ? k0 + k : 0) * a.ohead];
				for (int k = 0; k < 16 && k0 + k < a.nh; k++) acc = acc + b[k];
			}
			v[u] = v[u] + acc;
		}
	}
	for (int u = 0; u < NL_EPT; u++) {
		const int e = tid + u * NL_TPB, l = e >> ks, i = e & km;
		const bool in = L0 + l < a.lines && i < D;
		if (in && a.mode) a.h[lh[l] + i] = v[u];
		z[l * ZS + i] = in ? v[u] * v[u] : 0.0f;
	}
	__syncthreads();
	if (tid < R && L0 + tid < a.lines) linv[tid] = 1.0f / sqrtf(tg_ordered_sum_pp<6>(z + tid * ZS, D) / (float)D + 1e-6f);
	__syncthreads();
	{
		float gv[NL_EPT]; // the gains, all loaded before the first is used
		for (int u = 0; u < NL_EPT; u++) {
			const int e = tid + u * NL_TPB, l = e >> ks, i = e & km;
			gv[u] = a.g[lg[l] + (i < D ? i : D - 1)];
		}
		for (int u = 0; u < NL_EPT; u++) {
			const int e = tid + u * NL_TPB, l = e >> ks, i = e & km;
			const bool in = L0 + l < a.lines && i < D;
			float nv = 0.0f;
			if (in) {
				nv = v[u] * linv[l] * gv[u];
				a.out[(L0 + l) * D + i] = nv;
			}
			z[l * ZS + i] = nv;
		}
	}
	__syncthreads();
	// per line: TPL = NL_TPB / R consecutive lanes (within one wave) take its max
	// and flag, then its 16-input digit groups (Kp / 16 / TPL = 2 each) and
	// the sum of their q, combined by shuffles
	const int TPL = NL_TPB / R, l = tid / TPL, k = tid - l * TPL;
	const float *zl = z + l * ZS;
	float mx = 0.0f;
	int bad = 0;
	for (int m = k; m < Kp; m += TPL) {
		const float x = zl[m];
		bad |= !isfinite(x);
		mx = fmaxf(mx, fabsf(x)); // a nan never wins fmaxf; such lines are flagged
	}
	for (int o = 1; o < TPL; o <<= 1) {
		mx = fmaxf(mx, __shfl_xor(mx, o));
		bad |= __shfl_xor(bad, o);
	}
	const int special = tgq_special(bad, mx), E = tgq_exponent(mx, special);
	long long qs = 0, tl = 0;
	if (L0 + l < a.lines) {
		int8_t *blk = tgq_row_base(a.q.dig, (int)(L0 + l), Kp);
		for (int gi = k; gi < Kp / 16; gi += TPL) {
			float w16[16];
			for (int q = 0; q < 16; q++) w16[q] = zl[gi * 16 + q];
			qs += tgq_put16(blk, gi * 16, w16, E, special, tl);
		}
	}
	for (int o = 1; o < TPL; o <<= 1) qs += __shfl_xor(qs, o), tl += __shfl_xor(tl, o);
	int cls = special ? TGQ_REF : tgq_candidate(tl) ? TGQ_CAND : TGQ_GRID;
	TgqCoarse co{}; // the coarse test of candidate lines before any resolve (shuffles within the line's lanes)
	if (cls == TGQ_CAND)
		for (int gi = k; gi < Kp / 16; gi += TPL) {
			float w16[16];
			for (int q = 0; q < 16; q++) w16[q] = zl[gi * 16 + q];
			tgq_coarse16(co, w16, E);
		}
	for (int o = 1; o < TPL; o <<= 1)
		co.cnt += __shfl_xor(co.cnt, o), co.s0 += __shfl_xor(co.s0, o), co.s1 += __shfl_xor(co.s1, o);
	if (cls == TGQ_CAND && tgq_coarse_grid(co, tl)) cls = TGQ_GRID;
	if (k == 0 && L0 + l < a.lines) {
		const long L = L0 + l;
		a.q.e[L] = E, a.q.special[L] = cls, a.q.qsum[L] = qs;
	}
}

// tgk_dec_silu: one block per row; silu as the element-wise kernels compute it
__global__ __launch_bounds__(1024) void dec_silu_k(tgk_dec_silu_args a)
{
	extern __shared__ float4 zs4[]; // [Kp]
	float *zs = (float *)zs4;
	__shared__ float redf[16];
	__shared__ unsigned long long redl[5 * 16];
	const int t = blockIdx.x, FF = a.FF;
	const float *g = a.gu + (long)t * a.gus, *u = g + FF;
	float mx = 0.0f;
	int bad = 0;
	for (int i = threadIdx.x; i < a.Kp; i += blockDim.x) {
		float v = 0.0f;
		if (i < FF) {
			const float x = g[i];
			v = x / (1.0f + expf(-x)) * u[i];
			a.out[(long)t * FF + i] = v;
			bad |= !isfinite(v);
			mx = fmaxf(mx, fabsf(v));
		}
		zs[i] = v;
	}
	__syncthreads();
	blk_digits(zs, FF, a.Kp, mx, bad, a.q, t, redf, redl);
}

// out = silu(g) * u for a prompt's many rows [g (FF) | u (FF)] (gus apart),
// the operations dec_silu_k applies, streamed four values a thread (when FF,
// gus and the pointers allow 16-byte accesses); the GEMM's own digit kernel
// makes the digits after it. Block y takes rows y, y + gridDim.y, ...
__global__ __launch_bounds__(256) void silu_mul_k(const float *gu, long gus, float *out, int FF, int rows, int vec)
{
	const int i = (blockIdx.x * 256 + threadIdx.x) * 4;
	if (i >= FF) return;
	auto one = [](float x, float u) { return x / (1.0f + expf(-x)) * u; };
	for (int t = blockIdx.y; t < rows; t += gridDim.y) {
		const float *g = gu + (long)t * gus, *u = g + FF;
		float *o = out + (long)t * FF;
		if (vec) {
			const float4 gv = *(const float4 *)(g + i), uv = *(const float4 *)(u + i);
			*(float4 *)(o + i) = make_float4(one(gv.x, uv.x), one(gv.y, uv.y), one(gv.z, uv.z), one(gv.w, uv.w));
		} else
			for (int k = i; k < i + 4 && k < FF; k++) o[k] = one(g[k], u[k]);
	}
}

// A prompt chunk's causal softmax of one head's scores, line (sequence, t)
// of sc = q_t . k_u for u <= t (the products above the diagonal are not
// computed). The graph's operations on the valid part: x_u = s_u * scale + 0
// (the mask's 0), the row op's max rule, expf(x_u - max), the sum in key
// order, e_u / sum. Above the diagonal the graph adds -1e9: for finite scores
// that entry never wins the max and its expf is exactly 0, which leaves the
// sum unchanged and gives p_u = 0, written here directly. lpb lines per block
// (a power of two >= 4) staged in LDS, stride T0 + 4 floats (16-byte aligned).
__global__ __launch_bounds__(256) void causal_softmax_k(float *sc, int T0, long nlines, float scale, int lpb, int stride)
{
	extern __shared__ float4 sh4[];
	float *z = (float *)sh4, *lv = z + lpb * stride; // lv: per line max, then sum
	const long L0 = (long)blockIdx.x * lpb;
	const int tid = threadIdx.x, t0 = (int)(L0 % T0);
	const int nl = nlines - L0 < lpb ? (int)(nlines - L0) : lpb; // lines of this block
	auto pos = [&](int ll) { return (t0 + ll) % T0; };          // line ll's position t
	for (int ll = 0; ll < nl; ll++) {
		const int t = pos(ll);
		const float *src = sc + (L0 + ll) * T0;
		for (int u = tid; u <= t; u += 256) z[ll * stride + u] = src[u] * scale + 0.0f;
	}
	__syncthreads();
	{ // max: 256 / lpb consecutive lanes of one wave per line
		const int tpl = 256 / lpb, l = tid / tpl, sub = tid - l * tpl;
		const int t = l < nl ? pos(l) : 0;
		const float *y = z + l * stride;
		float m = -INFINITY;
		for (int u = 1 + sub; u <= t; u += tpl) m = fmaxf(m, y[u]);
		for (int w = tpl / 2; w > 0; w >>= 1) m = fmaxf(m, __shfl_xor(m, w));
		if (sub == 0) lv[l] = isnan(y[0]) ? y[0] : fmaxf(y[0], m);
	}
	__syncthreads();
	for (int ll = 0; ll < nl; ll++) {
		const int t = pos(ll);
		for (int u = tid; u <= t; u += 256) z[ll * stride + u] = expf(z[ll * stride + u] - lv[ll]);
	}
	__syncthreads();
	if (tid < nl) lv[tid] = tg_ordered_sum_pp<6>(z + tid * stride, pos(tid) + 1);
	__syncthreads();
	for (int ll = 0; ll < nl; ll++) {
		const int t = pos(ll);
		float *dst = sc + (L0 + ll) * T0;
		for (int u = tid; u < T0; u += 256) dst[u] = u <= t ? z[ll * stride + u] / lv[ll] : 0.0f;
	}
}

// Greedy choice per row: the index of the largest logit, the first one on
// ties, a nan counting as largest (numpy's argmax). (nan-ness, value, -index)
// is a total order, so any grouping of the comparisons finds the same index:
// argmax_part_k takes the best of each of a row's parts (blocks of `chunk`
// columns, loads in batches of 8 per thread), argmax_fin_k the best of the
// parts, written as an f32 token id (the model's input format) and as an int.
__device__ inline bool am_better(float a, int ia, float b, int ib) // is (a, ia) the better candidate?
{
	if (ib < 0) return ia >= 0;
	if (ia < 0) return false;
	const bool na = isnan(a), nb = isnan(b);
	if (na != nb) return na;
	if (!na && a != b) return a > b;
	return ia < ib;
}

__device__ inline void am_wave(float &v, int &i)
{
	for (int w = 32; w > 0; w >>= 1) {
		const float ov = __shfl_xor(v, w);
		const int oi = __shfl_xor(i, w);
		if (am_better(ov, oi, v, i)) v = ov, i = oi;
	}
}

__global__ __launch_bounds__(256) void argmax_part_k(const float *x, long xrs, int V, int chunk, int nparts, float *pv, int *pi)
{
	__shared__ float bv[4];
	__shared__ int bi[4];
	const int row = blockIdx.x / nparts, part = blockIdx.x - row * nparts;
	const float *r = x + (long)row * xrs;
	const int k0 = part * chunk, k1 = min(V, k0 + chunk);
	float v = 0.0f;
	int i = -1;
	for (int b = k0; b < k1; b += 8 * 256) {
		float u[8];
		for (int j = 0; j < 8; j++) {
			const int k = b + j * 256 + (int)threadIdx.x;
			u[j] = r[k < k1 ? k : k1 - 1];
		}
		for (int j = 0; j < 8; j++) {
			const int k = b + j * 256 + (int)threadIdx.x;
			if (k < k1 && am_better(u[j], k, v, i)) v = u[j], i = k;
		}
	}
	am_wave(v, i);
	if ((threadIdx.x & 63) == 0) bv[threadIdx.x >> 6] = v, bi[threadIdx.x >> 6] = i;
	__syncthreads();
	if (threadIdx.x == 0) {
		for (int w = 1; w < 4; w++)
			if (am_better(bv[w], bi[w], v, i)) v = bv[w], i = bi[w];
		pv[blockIdx.x] = v;
		pi[blockIdx.x] = i;
	}
}

__global__ __launch_bounds__(64) void argmax_fin_k(const float *pv, const int *pi, int nparts, float *idf, int *idi, long idi_stride)
{
	const int row = blockIdx.x, l = threadIdx.x;
	float v = l < nparts ? pv[(long)row * nparts + l] : 0.0f;
	int i = l < nparts ? pi[(long)row * nparts + l] : -1;
	am_wave(v, i);
	if (l == 0) {
		idf[row] = (float)i;
		if (idi) idi[(long)row * idi_stride] = i;
	}
}

constexpr int TPB = 256;
inline unsigned blocks(long n) { return (unsigned)((n + TPB - 1) / TPB); }

} // namespace

size_t tgk_dec_attn_lds(int GRP, int HD, int n)
{
	const long nst = (n + 3) & ~3;
	return (size_t)((long)attn_chunk(HD) * (HD + 4) + (long)GRP * HD + GRP * nst + GRP) * sizeof(float);
}


void tgk_dec_rope(hipStream_t s, const tgk_dec_rope_args *a, int rows)
{
	const long total = (long)rows * (a->NQ + 2 * a->NKV) * a->HD;
	if (total <= 0) return;
	auto al = [](const void *p) { return ((size_t)p & 15) == 0; };
	if (a->HD % 4 == 0 && a->ctot % 4 == 0 && a->kv_seq % 4 == 0 && a->kv_layer % 4 == 0 && al(a->hq) && al(a->rt) && al(a->qkv) &&
	    al(a->cosT) && al(a->sinT) && al(a->qr) && al(a->K) && al(a->V)) {
		const int per = (a->NQ + 2 * a->NKV) * (a->HD / 4);
		const dim3 grid((unsigned)((per + 255) / 256), (unsigned)(rows < 65535 ? rows : 65535));
		rope_cache4_k<<<grid, 256, 0, s>>>(*a, rows);
	} else
		rope_cache_k<<<blocks(total), TPB, 0, s>>>(*a, total);
}

void tgk_dec_attn(hipStream_t s, const tgk_dec_attn_args *a, int seqs)
{
	const int GRP = a->NQ / a->NKV, ck = attn_chunk(a->HD);
	const size_t lds = tgk_dec_attn_lds(GRP, a->HD, a->p + 1);
	const unsigned grid = (unsigned)(seqs * a->NKV);
	if (seqs <= 0) return;
	switch (GRP) { // the decoder checks GRP, HD and the LDS size when it is created
	case 1: dec_attn_k<1><<<grid, ATT_TPB, lds, s>>>(*a, ck); break;
	case 2: dec_attn_k<2><<<grid, ATT_TPB, lds, s>>>(*a, ck); break;
	case 4: dec_attn_k<4><<<grid, ATT_TPB, lds, s>>>(*a, ck); break;
	case 8: dec_attn_k<8><<<grid, ATT_TPB, lds, s>>>(*a, ck); break;
	default: break;
	}
}

// many lines (a prompt): norm_lines_k; few (a step): a block per row or a wave per head line
constexpr long NL_MIN_LINES = 2048;
inline bool nl_fits(int Kp) { return Kp >= 64 && Kp <= NL_E && (Kp & (Kp - 1)) == 0; } // a power of two: lines by shifts
inline int ilog2(int x) { int k = 0; while ((1 << (k + 1)) <= x) k++; return k; }

bool tgk_dec_norm(hipStream_t s, const tgk_dec_norm_args *a)
{
	if (a->rows <= 0) return true;
	if (a->rows >= NL_MIN_LINES && nl_fits(a->Kp) && a->outs == a->D) {
		NormLines n{ a->h, a->hs, a->mode, a->add, a->adds, a->o, a->ohead, a->nh, a->g, 0, a->out, a->D, a->Kp, 1, a->rows, a->q, ilog2(a->Kp) };
		const long R = NL_E / a->Kp;
		norm_lines_k<<<(unsigned)((a->rows + R - 1) / R), NL_TPB, norm_lines_lds(a->Kp), s>>>(n);
		return false; // candidates left for tgk_qgemm_split
	}
	dec_norm_k<<<(unsigned)a->rows, NORM_TPB, (size_t)a->Kp * 2 * sizeof(float), s>>>(*a);
	return true;
}

bool tgk_dec_hnorm(hipStream_t s, const tgk_dec_hnorm_args *a)
{
	const long lines = (long)a->rows * a->NH;
	if (lines <= 0) return true;
	if (lines >= NL_MIN_LINES && nl_fits(a->Kp)) {
		NormLines n{ (float *)a->x, a->xs, 0, nullptr, 0, nullptr, 0, 0, a->g, a->HD, a->out, a->HD, a->Kp, a->NH, lines, a->q, ilog2(a->Kp) };
		const long R = NL_E / a->Kp;
		norm_lines_k<<<(unsigned)((lines + R - 1) / R), NL_TPB, norm_lines_lds(a->Kp), s>>>(n);
		return false; // candidates left for tgk_qgemm_split
	}
	dec_hnorm_k<<<(unsigned)((lines + 3) / 4), TPB, (size_t)a->Kp * 8 * sizeof(float), s>>>(*a);
	return true;
}

void tgk_dec_silu_mul(hipStream_t s, const float *gu, long gus, float *out, int FF, int rows)
{
	if (rows <= 0 || FF <= 0) return;
	const int vec = FF % 4 == 0 && gus % 4 == 0 && ((size_t)gu & 15) == 0 && ((size_t)out & 15) == 0;
	const dim3 grid((unsigned)((FF + 1023) / 1024), (unsigned)(rows < 65535 ? rows : 65535));
	silu_mul_k<<<grid, 256, 0, s>>>(gu, gus, out, FF, rows, vec);
}

bool tgk_dec_silu(hipStream_t s, const tgk_dec_silu_args *a)
{
	if (a->rows > 0) dec_silu_k<<<(unsigned)a->rows, 1024, (size_t)a->Kp * sizeof(float), s>>>(*a);
	return true;
}

void tgk_dec_causal_softmax(hipStream_t s, float *sc, int T0, long nlines, float scale)
{
	if (nlines <= 0 || T0 <= 0) return;
	const int stride = (T0 + 3) / 4 * 4 + 4;
	int lpb = 64; // a power of two >= 4: lines per block
	while (lpb > 4 && (long)lpb * stride * 4 + lpb * 4 > 65536) lpb >>= 1;
	causal_softmax_k<<<(unsigned)((nlines + lpb - 1) / lpb), 256, (size_t)lpb * stride * 4 + lpb * 4, s>>>(sc, T0, nlines, scale, lpb, stride);
}

size_t tgk_dec_wo_lds(int rows, int HD)
{
	return (size_t)rows * HD * 4 + WO_NW * sizeof(TgqHist) + (size_t)rows * (8 + 8 * wo_nout(HD) + 8) + (size_t)HD * 64;
}

void tgk_dec_wo(hipStream_t s, const float *att, const int *codes, const float *scales, float *out, int rows, int NQ, int HD, int D)
{
	if (rows > 0) dec_wo_k<<<(unsigned)(NQ * ((D + 63) / 64)), WO_TPB, tgk_dec_wo_lds(rows, HD), s>>>(att, codes, scales, out, rows, NQ, HD, D);
}

void tgk_dec_argmax(hipStream_t s, const float *x, long xrs, int V, int rows, float *idf, int *idi, long idi_stride, float *pv, int *pi)
{
	if (rows <= 0 || V <= 0) return;
	const int np0 = (V + 2047) / 2048, nparts = np0 < TGK_AM_PARTS ? np0 : TGK_AM_PARTS, chunk = (V + nparts - 1) / nparts;
	argmax_part_k<<<(unsigned)(rows * nparts), TPB, 0, s>>>(x, xrs, V, chunk, nparts, pv, pi);
	argmax_fin_k<<<(unsigned)rows, 64, 0, s>>>(pv, pi, nparts, idf, idi, idi_stride);
}
