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
// sums.
__global__ __launch_bounds__(256) void dec_attn_k(tgk_dec_attn_args a)
{
	extern __shared__ float sh[];
	const int GRP = a.NQ / a.NKV, n = a.p + 1;
	const int s = blockIdx.x / a.NKV, j = blockIdx.x - s * a.NKV;
	float *sc = sh;                  // [GRP][n]
	float *q = sc + GRP * n;         // [GRP][HD]
	float *lv = q + GRP * a.HD;      // [GRP] max, then sum
	const float *K = a.K + (long)s * a.kv_seq + a.kv_layer + (long)j * a.P * a.HD;
	const float *V = a.V + (long)s * a.kv_seq + a.kv_layer + (long)j * a.P * a.HD;
	for (int e = threadIdx.x; e < GRP * a.HD; e += blockDim.x) q[e] = a.qr[((long)s * a.NQ + j * GRP) * a.HD + e];
	__syncthreads();
	for (int e = threadIdx.x; e < GRP * n; e += blockDim.x) {
		const int g = e / n, key = e - g * n;
		const float *kr = K + (long)key * a.HD, *qg = q + g * a.HD;
		float acc = 0.0f;
		for (int d = 0; d < a.HD; d++) acc = acc + qg[d] * kr[d];
		sc[e] = acc * a.scale + 0.0f;
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
	for (int e = threadIdx.x; e < GRP * a.HD; e += blockDim.x) {
		const int g = e / a.HD, d = e - g * a.HD;
		const float *r = sc + g * n;
		float acc = 0.0f;
		for (int key = 0; key < n; key++) acc = acc + r[key] * V[(long)key * a.HD + d];
		a.att[((long)s * a.NQ + j * GRP + g) * a.HD + d] = acc;
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
	if (seqs > 0) dec_attn_k<<<(unsigned)(seqs * a->NKV), TPB, lds, s>>>(*a);
}

void tgk_dec_sumchain(hipStream_t s, float *h, const float *o, int NQ, long per_head)
{
	if (per_head > 0) sumchain_k<<<blocks(per_head), TPB, 0, s>>>(h, o, NQ, per_head, per_head);
}

void tgk_dec_argmax(hipStream_t s, const float *x, long xrs, int V, int rows, float *idf, int *idi, long idi_stride)
{
	if (rows > 0) argmax_k<<<(unsigned)rows, TPB, 0, s>>>(x, xrs, V, idf, idi, idi_stride);
}
