// Kernels of the KV-cache decoder (tg_decode.cpp) for models in the Qwen3
// importer's layout (examples/qwen3/import.py). Each computes the values the
// fixed-length graph computes, with the same f32 operations in the same
// order (this file is compiled with -ffp-contract=off), so a decoded token's
// logits equal the fixed-length forward's at that position bit for bit.
#include "tg_kern.h"

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

// One decode step's attention: one block per (sequence, KV head) for the GRP
// query heads sharing it, keys at positions 0 .. p. Per query head and key:
// score = sum_d q[d] k[d] in order from 0.0f, times the scale, plus the mask's
// 0; softmax with the reference's max rule, expf, a sequential sum and a
// division; out[d] = sum over keys of prob * v[d] in key order. The
// fixed-length graph's row for this position has further keys whose masked
// scores give probabilities of exactly 0: they change neither the max nor the
// sums. A thread takes one key for all GRP query heads (K read once, GRP
// independent chains) and loads its K values 16 at a time before the ordered
// multiply-adds; the P V chain of each (head, d) loads 8 keys ahead. Every
// score and every output stays one thread's sum in order. HD % 16 == 0.
template <int GRP>
__global__ __launch_bounds__(256) void dec_attn_k(tgk_dec_attn_args a)
{
	extern __shared__ float sh[];
	const int n = a.p + 1, HD = a.HD;
	const int s = blockIdx.x / a.NKV, j = blockIdx.x - s * a.NKV;
	float *sc = sh;          // [GRP][n]
	float *q = sc + GRP * n; // [GRP][HD]
	float *lv = q + GRP * HD; // [GRP] max, then sum
	const float *K = a.K + (long)s * a.kv_seq + a.kv_layer + (long)j * a.P * HD;
	const float *V = a.V + (long)s * a.kv_seq + a.kv_layer + (long)j * a.P * HD;
	for (int e = threadIdx.x; e < GRP * HD; e += blockDim.x) q[e] = a.qr[((long)s * a.NQ + j * GRP) * HD + e];
	__syncthreads();
	for (int key = threadIdx.x; key < n; key += blockDim.x) {
		const float4 *kr = (const float4 *)(K + (long)key * HD);
		float acc[GRP];
		for (int g = 0; g < GRP; g++) acc[g] = 0.0f;
		for (int d0 = 0; d0 < HD; d0 += 16) {
			float k[16];
			for (int u = 0; u < 4; u++) {
				const float4 v = kr[d0 / 4 + u];
				k[4 * u] = v.x, k[4 * u + 1] = v.y, k[4 * u + 2] = v.z, k[4 * u + 3] = v.w;
			}
			for (int dd = 0; dd < 16; dd++)
				for (int g = 0; g < GRP; g++) acc[g] = acc[g] + q[g * HD + d0 + dd] * k[dd];
		}
		for (int g = 0; g < GRP; g++) sc[g * n + key] = acc[g] * a.scale + 0.0f;
	}
	__syncthreads();
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
	for (int g = wave; g < GRP; g += blockDim.x >> 6) { // max: a wave per query head
		const float *r = sc + g * n;
		float m = -INFINITY;
		for (int key = 1 + lane; key < n; key += 64) m = fmaxf(m, r[key]);
		for (int w = 32; w > 0; w >>= 1) m = fmaxf(m, __shfl_xor(m, w));
		if (lane == 0) lv[g] = isnan(r[0]) ? r[0] : fmaxf(r[0], m);
	}
	__syncthreads();
	for (int e = threadIdx.x; e < GRP * n; e += blockDim.x) sc[e] = expf(sc[e] - lv[e / n]);
	__syncthreads();
	if ((int)threadIdx.x < GRP) {
		const float *r = sc + threadIdx.x * n;
		float sum = 0.0f;
		for (int key = 0; key < n; key++) sum += r[key];
		lv[threadIdx.x] = sum;
	}
	__syncthreads();
	for (int e = threadIdx.x; e < GRP * n; e += blockDim.x) sc[e] = sc[e] / lv[e / n];
	__syncthreads();
	for (int e = threadIdx.x; e < GRP * HD; e += blockDim.x) {
		const int g = e / HD, d = e - g * HD;
		const float *r = sc + g * n;
		const float *vp = V + d;
		float acc = 0.0f;
		int key = 0;
		for (; key + 8 <= n; key += 8) {
			float v[8];
			for (int u = 0; u < 8; u++) v[u] = vp[(long)(key + u) * HD];
			for (int u = 0; u < 8; u++) acc = acc + r[key + u] * v[u];
		}
		for (; key < n; key++) acc = acc + r[key] * vp[(long)key * HD];
		a.att[((long)s * a.NQ + j * GRP + g) * HD + d] = acc;
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
// 2^100 take the reference's sequential f32 loop. One block per (head, 64
// columns): the rows' digits and the head's code tile sit in LDS; a wave
// handles 4 rows at a time, a lane one column.
// codes: int32 [NQ][HD/4][D], 4 consecutive k's int8 codes per word (k = 4
// k4 + i in byte i); scales [NQ][D]; HD a multiple of 4.
__global__ __launch_bounds__(256) void dec_wo_k(const float *att, const int *codes, const float *scales, float *out, int rows, int NQ,
						int HD, int D)
{
	extern __shared__ int4 dg[]; // [rows][HD/4] digit words {d0, d1, d2, 0} of 4 k's
	const int H4 = HD / 4;
	int *Es = (int *)(dg + (long)rows * H4), *sp = Es + rows, *ct = sp + rows; // ct: [HD/4][64] code words
	const int ctiles = (D + 63) / 64, g = blockIdx.x / ctiles, c0 = (blockIdx.x - g * ctiles) * 64;
	const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
	for (int t = wave; t < rows; t += nw) { // a wave per token row
		const float *x = att + ((long)t * NQ + g) * HD;
		float mx = 0.0f;
		int bad = 0;
		for (int k = lane; k < HD; k += 64) {
			bad |= !isfinite(x[k]);
			mx = fmaxf(mx, fabsf(x[k]));
		}
		for (int w = 32; w > 0; w >>= 1) {
			mx = fmaxf(mx, __shfl_xor(mx, w));
			bad |= __shfl_xor(bad, w);
		}
		const int special = bad || mx > 0x1p100f;
		int E = 0;
		if (!special && mx > 0.0f) {
			frexpf(mx, &E);
			if (rintf(ldexpf(mx, 23 - E)) > 8355328.0f) E += 1;
		}
		for (int k4 = lane; k4 < H4; k4 += 64) {
			unsigned w0 = 0, w1 = 0, w2 = 0;
			if (!special)
				for (int i = 0; i < 4; i++) {
					const int q = (int)rintf(ldexpf(x[4 * k4 + i], 23 - E)); // exact: |q| < 2^23
					const int d0 = (int)(int8_t)(q & 255), q1 = (q - d0) >> 8;
					const int d1 = (int)(int8_t)(q1 & 255), d2 = (q1 - d1) >> 8;
					w0 |= (unsigned)(d0 & 255) << (8 * i);
					w1 |= (unsigned)(d1 & 255) << (8 * i);
					w2 |= (unsigned)(d2 & 255) << (8 * i);
				}
			dg[(long)t * H4 + k4] = make_int4((int)w0, (int)w1, (int)w2, 0);
		}
		if (lane == 0) Es[t] = E, sp[t] = special;
	}
	for (int e = threadIdx.x; e < H4 * 64; e += blockDim.x) {
		const int k4 = e >> 6, c = e & 63;
		ct[e] = c0 + c < D ? codes[((long)g * H4 + k4) * D + c0 + c] : 0;
	}
	__syncthreads();
	const int c = lane;
	if (c0 + c >= D) return;
	const float sc = scales[(long)g * D + c0 + c];
	for (int t0 = 4 * wave; t0 < rows; t0 += 4 * nw) {
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
			float v;
			if (sp[t]) { // the reference's loop (runtime/tg_rt.h:143-151)
				const float *x = att + ((long)t * NQ + g) * HD;
				float acc = 0.0f;
				for (int k = 0; k < HD; k++) acc += (float)(int8_t)(ct[(k >> 2) * 64 + c] >> (8 * (k & 3))) * x[k];
				v = acc;
			} else { // every term and partial sum an integer below 2^48: exact in f64
				const double tot = (double)s[r][0] + (double)s[r][1] * 256.0 + (double)s[r][2] * 65536.0;
				v = (float)ldexp(tot, Es[t] - 23);
			}
			out[((long)g * rows + t) * D + c0 + c] = sc * v;
		}
	}
}

// h = h + ((o_0 + o_1) + ... + o_{NQ-1}): the graph's sum of the per-head
// output projections, then the residual add
__global__ void sumchain_k(float *h, const float *o, int NQ, long per_head, long total)
{
	const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
	if (t >= total) return;
	float acc = o[t];
	for (int k = 1; k < NQ; k++) acc = acc + o[(long)k * per_head + t];
	h[t] = h[t] + acc;
}

// Greedy choice per row: the index of the largest logit, the first one on
// ties, a nan counting as largest (numpy's argmax). Written as an f32 token id
// (the model's input format) and as an int.
__global__ __launch_bounds__(256) void argmax_k(const float *x, long xrs, int V, float *idf, int *idi, long idi_stride)
{
	__shared__ float bv[256];
	__shared__ int bi[256];
	const float *r = x + (long)blockIdx.x * xrs;
	float v = 0.0f;
	int i = -1;
	auto better = [](float a, int ia, float b, int ib) { // is (a, ia) the better candidate?
		if (ib < 0) return ia >= 0;
		if (ia < 0) return false;
		const bool na = isnan(a), nb = isnan(b);
		if (na != nb) return na;
		if (!na && a != b) return a > b;
		return ia < ib;
	};
	for (int k = threadIdx.x; k < V; k += blockDim.x)
		if (better(r[k], k, v, i)) v = r[k], i = k;
	bv[threadIdx.x] = v;
	bi[threadIdx.x] = i;
	__syncthreads();
	for (int w = blockDim.x / 2; w > 0; w >>= 1) {
		if ((int)threadIdx.x < w && better(bv[threadIdx.x + w], bi[threadIdx.x + w], bv[threadIdx.x], bi[threadIdx.x])) {
			bv[threadIdx.x] = bv[threadIdx.x + w];
			bi[threadIdx.x] = bi[threadIdx.x + w];
		}
		__syncthreads();
	}
	if (threadIdx.x == 0) {
		idf[blockIdx.x] = (float)bi[0];
		if (idi) idi[(long)blockIdx.x * idi_stride] = bi[0];
	}
}

constexpr int TPB = 256;
inline unsigned blocks(long n) { return (unsigned)((n + TPB - 1) / TPB); }

} // namespace

void tgk_dec_rope(hipStream_t s, const tgk_dec_rope_args *a, int rows)
{
	const long total = (long)rows * (a->NQ + 2 * a->NKV) * a->HD;
	if (total > 0) rope_cache_k<<<blocks(total), TPB, 0, s>>>(*a, total);
}

void tgk_dec_attn(hipStream_t s, const tgk_dec_attn_args *a, int seqs)
{
	const int GRP = a->NQ / a->NKV;
	const size_t lds = ((size_t)GRP * (a->p + 1) + (size_t)GRP * a->HD + GRP) * sizeof(float);
	const unsigned grid = (unsigned)(seqs * a->NKV);
	if (seqs <= 0) return;
	switch (GRP) { // the decoder checks GRP and HD when it is created
	case 1: dec_attn_k<1><<<grid, TPB, lds, s>>>(*a); break;
	case 2: dec_attn_k<2><<<grid, TPB, lds, s>>>(*a); break;
	case 4: dec_attn_k<4><<<grid, TPB, lds, s>>>(*a); break;
	case 8: dec_attn_k<8><<<grid, TPB, lds, s>>>(*a); break;
	default: break;
	}
}

size_t tgk_dec_wo_lds(int rows, int HD) { return (size_t)rows * HD * 4 + (size_t)rows * 8 + (size_t)HD * 64; }

void tgk_dec_wo(hipStream_t s, const float *att, const int *codes, const float *scales, float *out, int rows, int NQ, int HD, int D)
{
	if (rows > 0) dec_wo_k<<<(unsigned)(NQ * ((D + 63) / 64)), TPB, tgk_dec_wo_lds(rows, HD), s>>>(att, codes, scales, out, rows, NQ, HD, D);
}

void tgk_dec_sumchain(hipStream_t s, float *h, const float *o, int NQ, long per_head)
{
	if (per_head > 0) sumchain_k<<<blocks(per_head), TPB, 0, s>>>(h, o, NQ, per_head, per_head);
}

void tgk_dec_argmax(hipStream_t s, const float *x, long xrs, int V, int rows, float *idf, int *idi, long idi_stride)
{
	if (rows > 0) argmax_k<<<(unsigned)rows, TPB, 0, s>>>(x, xrs, V, idf, idi, idi_stride);
}
