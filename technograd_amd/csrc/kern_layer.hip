// Layer-executor kernels: one launch per model instruction over a block of
// batch rows. Values of a batch live as [rows][numel] in one device arena;
// params and constants are shared by all rows (row stride 0).
//
// Arithmetic follows the reference kernels (runtime/tg_rt.h) operation for
// operation: the same expression shapes, sums in index order from 0.0f,
// separate multiply and add (this file is compiled with -ffp-contract=off),
// correctly rounded division and square root. Transcendentals come from the
// ROCm device library, so only they differ from glibc (by a few ulp); the
// log1pf of softplus is this backend's own (tg_devmath.h), correctly rounded.
#include "tg_devmath.h"
#include "tg_ewop.h"
#include "tg_kern.h"
#include "tgm.h"

#include <math.h>

namespace {

constexpr int TPB = 256;

inline unsigned blocks_for(long n) { return (unsigned)((n + TPB - 1) / TPB); }

__device__ inline float bop(int op, float x, float y) { return tg_bop(op, x, y); }

// operand index of output element i (modes of tgk_binary)
__device__ inline int bidx(int mode, int i, const int *map, int per)
{
	return mode == 0 ? i : mode == 1 ? 0 : mode == 3 ? i % per : map[i];
}

__global__ void binary_k(int op, float *o, long ors, int n, tgk_opd a, int am, const int *amap, int aper, tgk_opd b, int bm,
			 const int *bmap, int bper, long total)
{
	long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
	if (t >= total) return;
	long r = t / n;
	int i = (int)(t - r * n);
	int ia = bidx(am, i, amap, aper);
	int ib = bidx(bm, i, bmap, bper);
	o[r * ors + i] = bop(op, a.p[r * a.rs + ia], b.p[r * b.rs + ib]);
}

// tg_rt.h:40-75
__device__ inline float uop(int op, float x) { return tg_uop(op, x); }

__global__ void unary_k(int op, float *o, long ors, tgk_opd a, int n, long total)
{
	long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
	if (t >= total) return;
	long r = t / n;
	int i = (int)(t - r * n);
	o[r * ors + i] = uop(op, a.p[r * a.rs + i]);
}

// Rows of at least ROWK elements: the grid is rows x chunks of EPT * TPB
// elements, so a thread finds its row with one division of the block index
// (the same for the whole block) instead of a 64-bit division per element.
// Each thread handles EPT elements TPB apart: its loads are all issued before
// the first result is stored.
constexpr int EPT = 4, ROWK = 512;

template <int OP>
__global__ __launch_bounds__(256) void binary_rows_k(float *o, long ors, int n, tgk_opd a, int am, const int *amap, int aper, tgk_opd b,
						     int bm, const int *bmap, int bper, int cpr)
{
	const int r = blockIdx.x / cpr;
	const int i0 = (blockIdx.x - r * cpr) * (TPB * EPT) + threadIdx.x;
	const float *ap = a.p + (long)r * a.rs, *bp = b.p + (long)r * b.rs;
	float x[EPT], y[EPT];
	for (int j = 0; j < EPT; j++) {
		const int i = i0 + j * TPB, ic = i < n ? i : n - 1;
		x[j] = ap[bidx(am, ic, amap, aper)];
		y[j] = bp[bidx(bm, ic, bmap, bper)];
	}
	float *op = o + (long)r * ors;
	for (int j = 0; j < EPT; j++) {
		const int i = i0 + j * TPB;
		if (i < n) op[i] = bop(OP, x[j], y[j]);
	}
}

// Both operands elementwise, rows 16-byte aligned, n a multiple of 4: EPT
// float4s per thread, TPB float4s apart.
template <int OP>
__global__ __launch_bounds__(256) void binary_rows4_k(float *o, long ors, int n, tgk_opd a, tgk_opd b, int cpr)
{
	const int r = blockIdx.x / cpr;
	const int i0 = ((blockIdx.x - r * cpr) * (TPB * EPT) + threadIdx.x) * 4;
	const float *ap = a.p + (long)r * a.rs, *bp = b.p + (long)r * b.rs;
	float4 x[EPT], y[EPT];
	for (int j = 0; j < EPT; j++) {
		const int i = i0 + j * TPB * 4, ic = i < n ? i : 0;
		x[j] = *(const float4 *)(ap + ic);
		y[j] = *(const float4 *)(bp + ic);
	}
	float *op = o + (long)r * ors;
	for (int j = 0; j < EPT; j++) {
		const int i = i0 + j * TPB * 4;
		if (i < n)
			*(float4 *)(op + i) = make_float4(bop(OP, x[j].x, y[j].x), bop(OP, x[j].y, y[j].y), bop(OP, x[j].z, y[j].z),
							  bop(OP, x[j].w, y[j].w));
	}
}

template <int OP>
__global__ __launch_bounds__(256) void unary_rows_k(float *o, long ors, tgk_opd a, int n, int cpr)
{
	const int r = blockIdx.x / cpr;
	const int i0 = (blockIdx.x - r * cpr) * (TPB * EPT) + threadIdx.x;
	const float *ap = a.p + (long)r * a.rs;
	float x[EPT];
	for (int j = 0; j < EPT; j++) {
		const int i = i0 + j * TPB;
		x[j] = ap[i < n ? i : n - 1];
	}
	float *op = o + (long)r * ors;
	for (int j = 0; j < EPT; j++) {
		const int i = i0 + j * TPB;
		if (i < n) op[i] = uop(OP, x[j]);
	}
}

template <int OP>
__global__ __launch_bounds__(256) void unary_rows4_k(float *o, long ors, tgk_opd a, int n, int cpr)
{
	const int r = blockIdx.x / cpr;
	const int i0 = ((blockIdx.x - r * cpr) * (TPB * EPT) + threadIdx.x) * 4;
	const float *ap = a.p + (long)r * a.rs;
	float4 x[EPT];
	for (int j = 0; j < EPT; j++) {
		const int i = i0 + j * TPB * 4;
		x[j] = *(const float4 *)(ap + (i < n ? i : 0));
	}
	float *op = o + (long)r * ors;
	for (int j = 0; j < EPT; j++) {
		const int i = i0 + j * TPB * 4;
		if (i < n) *(float4 *)(op + i) = make_float4(uop(OP, x[j].x), uop(OP, x[j].y), uop(OP, x[j].z), uop(OP, x[j].w));
	}
}

inline bool al16(const void *p, long rs) { return ((size_t)p & 15) == 0 && rs % 4 == 0; }

// A fused elementwise run (tgk_ew): four consecutive elements per thread.
// The N0 elementwise (or aligned whole-row repeat) inputs, the first ones, are
// loaded as straight-line float4 loads, all in flight together, then the
// others. The instruction list, the same for every thread, drives an
// accumulator (a float4 in VGPRs); the register file lives in LDS, one
// 16-byte slot per register and thread, which only that thread touches (no
// barriers). Kept in VGPRs, a register file indexed by run-time register
// numbers is copied whole at every loop iteration. Each instruction is the
// operation of binary_k or unary_k, so the stored values are bit-identical to
// running the instructions one launch at a time. VEC: the float4 inputs and
// all outputs are 16-byte aligned rows and n is a multiple of 4; otherwise N0
// is 0 and every input takes the general path.
__device__ inline void ew_gather(const tgk_ew &E, int j, int r, int i0, int n, float *v)
{
	const float *p = E.in[j] + (long)r * E.in_rs[j];
	const int mode = E.in_mode[j];
	if (mode == 1) {
		const float x = p[0];
		for (int e = 0; e < 4; e++) v[e] = x;
	} else {
		for (int e = 0; e < 4; e++) {
			const int ic = i0 + e < n ? i0 + e : n - 1;
			v[e] = p[bidx(mode, ic, E.in_map[j], E.in_per[j])];
		}
	}
}

template <int N0, bool VEC>
__global__ __launch_bounds__(256) void ew_k(tgk_ew E, int n, int cpr)
{
	__shared__ float4 R[TGK_EW_REGS][TPB];
	const int r = blockIdx.x / cpr;
	const int i0 = ((blockIdx.x - r * cpr) * TPB + threadIdx.x) * 4;
	float4 v0[N0 > 0 ? N0 : 1];
	for (int j = 0; j < N0; j++) { // mode 0, or mode 3 with a period that is a multiple of 4
		int idx = i0 < n ? i0 : 0;
		if (E.in_mode[j] == 3) {
			// idx mod per from a float quotient estimate: with fewer than 2^22
			// repeats the estimate is off by at most one, which the two
			// corrections absorb
			const int per = E.in_per[j];
			const int q = (int)((float)idx * E.in_inv[j]);
			int rr = idx - q * per;
			rr = rr < 0 ? rr + per : rr;
			idx = rr >= per ? rr - per : rr;
		}
		v0[j] = *(const float4 *)(E.in[j] + (long)r * E.in_rs[j] + idx);
	}
	for (int j = 0; j < N0; j++) R[j][threadIdx.x] = v0[j];
	for (int j = N0; j < TGK_EW_MAXIN; j++) // argument indices stay compile-time constants
		if (j < E.nin) {
			float g[4];
			ew_gather(E, j, r, i0, n, g);
			R[j][threadIdx.x] = make_float4(g[0], g[1], g[2], g[3]);
		}
	float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
	for (int k = 0; k < E.nins; k++) {
		const tgk_ew_ins I = E.ins[k];
		switch (I.kind) {
		case TGK_EW_LOAD: acc = R[I.a][threadIdx.x]; break;
		case TGK_EW_SAVE: R[I.dst][threadIdx.x] = acc; break;
		case TGK_EW_BIN: case TGK_EW_BINR: {
			const float4 o = R[I.a][threadIdx.x];
			const float4 x = I.kind == TGK_EW_BIN ? acc : o, y = I.kind == TGK_EW_BIN ? o : acc;
			switch (I.op) { // the op outside the element loop: each case is straight-line code
#define EWB(K) \
	case K: acc = make_float4(bop(K, x.x, y.x), bop(K, x.y, y.y), bop(K, x.z, y.z), bop(K, x.w, y.w)); break;
				EWB(TGK_ADD) EWB(TGK_SUB) EWB(TGK_MUL) EWB(TGK_DIV) EWB(TGK_MAX) EWB(TGK_MIN)
#undef EWB
			}
			break;
		}
		case TGK_EW_UN:
			switch (I.op) {
#define EWU(K) \
	case K: acc = make_float4(uop(K, acc.x), uop(K, acc.y), uop(K, acc.z), uop(K, acc.w)); break;
				EWU(TGM_NEG) EWU(TGM_TANH) EWU(TGM_RELU) EWU(TGM_SIGMOID) EWU(TGM_EXP) EWU(TGM_SQRT) EWU(TGM_GELU)
				EWU(TGM_SILU) EWU(TGM_SOFTPLUS) EWU(TGM_LOG) EWU(TGM_SIN) EWU(TGM_COS) EWU(TGM_FLOOR) EWU(TGM_STEP)
#undef EWU
			}
			break;
		default: { // TGK_EW_STORE
			float *p = E.out[I.dst] + (long)r * E.out_rs[I.dst];
			if (VEC) {
				if (i0 < n) *(float4 *)(p + i0) = acc;
			} else {
				const float a4[4] = { acc.x, acc.y, acc.z, acc.w };
				for (int e = 0; e < 4; e++)
					if (i0 + e < n) p[i0 + e] = a4[e];
			}
		}
		}
	}
}

__device__ inline int code_at(const uint8_t *q, int bits, long i)
{
	if (bits == 8) return (signed char)q[i];
	int b = (signed char)q[i >> 1];
	return (i & 1) ? (b >> 4) : (int)(signed char)(unsigned char)((unsigned)b << 4) >> 4;
}

__global__ void mm_exact_k(tgk_mm d, long total)
{
	long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
	if (t >= total) return;
	int j = (int)(t % d.n);
	long u = t / d.n;
	int i = (int)(u % d.m);
	u /= d.m;
	int g = (int)(u % d.g);
	long r = u / d.g;
	const float *A = d.a.p + r * d.a.rs + g * d.ag + i * d.ai;
	const float *B = d.b.p + r * d.b.rs + g * d.bg + (long)j * d.bj;
	float acc = 0.0f;
	if (d.quant == 1) {
		long base = (long)g * d.m * d.k + (long)i * d.k;
		for (int p = 0; p < d.k; p++) acc += (float)code_at(d.codes, d.bits, base + p) * B[p * d.bp];
		acc = d.scale[i] * acc;
	} else if (d.quant == 2) {
		for (int p = 0; p < d.k; p++) acc += A[p * d.ap] * (float)code_at(d.codes, d.bits, (long)p * d.n + j);
		acc = d.scale[j] * acc;
	} else {
		for (int p = 0; p < d.k; p++) acc += A[p * d.ap] * B[p * d.bp];
	}
	d.o[r * d.ors + g * d.og + i * d.oi + (long)j * d.oj] = acc;
}

// tg_rt.h:154-175
__global__ void rowop_k(int op, float *o, long ors, tgk_opd a, int nrow, int cols, long total)
{
	long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
	if (t >= total) return;
	long r = t / nrow;
	int q = (int)(t - r * nrow);
	const float *x = a.p + r * a.rs + (long)q * cols;
	float *y = o + r * ors + (long)q * cols;
	if (op == TGM_SOFTMAX) {
		float mx = x[0], s = 0.0f;
		for (int i = 1; i < cols; i++)
			if (x[i] > mx) mx = x[i];
		for (int i = 0; i < cols; i++) {
			y[i] = expf(x[i] - mx);
			s += y[i];
		}
		for (int i = 0; i < cols; i++) y[i] /= s;
	} else {
		float s = 0.0f;
		for (int i = 0; i < cols; i++) s += x[i] * x[i];
		float inv = 1.0f / sqrtf(s / (float)cols + 1e-6f);
		for (int i = 0; i < cols; i++) y[i] = x[i] * inv;
	}
}

// The same per-line results with the lines staged through LDS: a block takes
// lpb consecutive lines of one batch row (lpb divides nrow), which are
// contiguous in memory, so loads and stores are coalesced. Only the sums
// keep one thread per line, walking its line in the reference's order; the
// max, the exponentials, the division and the rmsnorm scaling are
// elementwise or order-free and use every thread. LDS lines are `stride`
// floats apart, stride odd, so the sequential walks fall in distinct banks.
// Softmax's max: x[0] when it is nan, else the largest of x[0] and the
// non-nan x[i] (the reference's `if (x[i] > mx) mx = x[i]`); its sign of zero
// cannot change expf(x - mx).
// sum_i z_i in index order, as the reference's loop: one thread, one add
// after another (tg_ordered_sum when the line is 16-byte aligned)
template <bool SQ = false>
__device__ inline float line_sum(const float *z, int cols)
{
	if ((((size_t)z) & 15) == 0) return tg_ordered_sum_pp<6, SQ>(z, cols);
	float sum = 0.0f;
	for (int i = 0; i < cols; i++) sum += SQ ? z[i] * z[i] : z[i];
	return sum;
}

__global__ __launch_bounds__(256) void rowop_lds_k(int op, float *o, long ors, tgk_opd a, int nrow, int cols, int lpb, int stride)
{
	extern __shared__ float lds[];
	float *lv = lds + lpb * stride; // one value per line (max, then sum or inverse rms)
	const int bpr = nrow / lpb, r = blockIdx.x / bpr, q0 = (blockIdx.x - r * bpr) * lpb;
	const int tot = lpb * cols;
	const float *x = a.p + (long)r * a.rs + (long)q0 * cols;
	// element e of the tile is line e / cols, column e % cols: a thread's
	// elements e, e + TPB, ... are walked by adding TPB as (dl lines, dc
	// columns), with one carry, instead of a division per element
	const int dl = TPB / cols, dc = TPB - dl * cols, l0 = (int)threadIdx.x / cols, c0 = (int)threadIdx.x - l0 * cols;
	auto step = [&](int &l, int &c) {
		l += dl, c += dc;
		if (c >= cols) c -= cols, l++;
	};
	constexpr int U = 8;
	{
		int l = l0, c = c0;
		for (int e0 = 0; e0 < tot; e0 += U * TPB) {
			float v[U];
			for (int j = 0; j < U; j++) {
				const int e = e0 + j * TPB + threadIdx.x;
				v[j] = x[e < tot ? e : tot - 1];
			}
			for (int j = 0; j < U; j++) {
				const int e = e0 + j * TPB + threadIdx.x;
				if (e < tot) lds[l * stride + c] = v[j];
				step(l, c);
			}
		}
	}
	__syncthreads();
	if (op == TGM_SOFTMAX) {
		// max: TPB / lpb threads per line, consecutive lanes of one wave (lpb >= 4)
		const int tpl = TPB / lpb, l = threadIdx.x / tpl, sub = threadIdx.x - l * tpl;
		float m = -INFINITY;
		const float *y = lds + l * stride;
		for (int i = 1 + sub; i < cols; i += tpl) m = fmaxf(m, y[i]);
		for (int w = tpl / 2; w > 0; w >>= 1) m = fmaxf(m, __shfl_xor(m, w));
		if (sub == 0) lv[l] = isnan(y[0]) ? y[0] : fmaxf(y[0], m);
		__syncthreads();
		for (int e = threadIdx.x, ll = l0, c = c0; e < tot; e += TPB, step(ll, c)) {
			float *z = lds + ll * stride + c;
			*z = expf(*z - lv[ll]);
		}
		__syncthreads();
		if ((int)threadIdx.x < lpb) lv[threadIdx.x] = line_sum(lds + threadIdx.x * stride, cols);
		__syncthreads();
		for (int e = threadIdx.x, ll = l0, c = c0; e < tot; e += TPB, step(ll, c)) {
			float *z = lds + ll * stride + c;
			*z = *z / lv[ll];
		}
	} else {
		// each square is formed as its value arrives, off the ordered chain of adds
		if ((int)threadIdx.x < lpb) lv[threadIdx.x] = 1.0f / sqrtf(line_sum<true>(lds + threadIdx.x * stride, cols) / (float)cols + 1e-6f);
		__syncthreads();
		for (int e = threadIdx.x, ll = l0, c = c0; e < tot; e += TPB, step(ll, c)) {
			float *z = lds + ll * stride + c;
			*z = *z * lv[ll];
		}
	}
	__syncthreads();
	float *out = o + (long)r * ors + (long)q0 * cols;
	for (int e = threadIdx.x, ll = l0, c = c0; e < tot; e += TPB, step(ll, c)) out[e] = lds[ll * stride + c];
}

// sum / mean of each row, one thread per row adding in index order (the
// reference's sequential f32 loop); a 16-byte aligned row is read with float4
// loads issued ahead of the adds (tg_ordered_sum), others one float at a time
__global__ void reduce_k(int op, float *o, long ors, tgk_opd a, int n, int rows)
{
	int r = blockIdx.x * blockDim.x + threadIdx.x;
	if (r >= rows) return;
	const float *x = a.p + (long)r * a.rs;
	float s = 0.0f;
	if (((size_t)x & 15) == 0) s = tg_ordered_sum_pp<6>(x, n);
	else
		for (int i = 0; i < n; i++) s += x[i];
	o[(long)r * ors] = op == TGM_SUM ? s : s / (float)n;
}

__global__ void transpose_k(float *o, long ors, tgk_opd a, int g, int R, int C, long total)
{
	long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
	if (t >= total) return;
	long per = (long)g * R * C;
	long r = t / per, e = t - r * per;
	int z = (int)(e / ((long)R * C)), rem = (int)(e % ((long)R * C)), i = rem / C, j = rem % C;
	o[r * ors + (long)z * R * C + (long)j * R + i] = a.p[r * a.rs + e];
}

__global__ void outer_k(float *o, long ors, tgk_opd a, int m, tgk_opd b, int n, long total)
{
	long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
	if (t >= total) return;
	long per = (long)m * n, r = t / per;
	int e = (int)(t - r * per), i = e / n, j = e % n;
	o[r * ors + e] = a.p[r * a.rs + i] * b.p[r * b.rs + j];
}

// tg_rt.h:200-204 (index rounding) and :316-323
__global__ void take_k(float *o, long ors, tgk_opd w, tgk_opd idx, int cnt, int d, int h, long total)
{
	long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
	if (t >= total) return;
	long per = (long)cnt * h, r = t / per;
	int e = (int)(t - r * per), i = e / h, j = e % h;
	float rr = floorf(idx.p[r * idx.rs + i] + 0.5f);
	int row = rr >= 0.0f && rr < (float)d ? (int)rr : -1;
	o[r * ors + e] = row >= 0 ? w.p[r * w.rs + (long)row * h + j] : 0.0f;
}

__global__ void copy_k(float *o, long ors, long ooff, tgk_opd a, long aoff, int w, long total)
{
	long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
	if (t >= total) return;
	long r = t / w;
	int i = (int)(t - r * w);
	o[r * ors + ooff + i] = a.p[r * a.rs + aoff + i];
}

} // namespace

void tgk_binary(hipStream_t s, int op, float *o, long ors, int n, tgk_opd a, int amode, const int *amap, int aper, tgk_opd b, int bmode,
		const int *bmap, int bper, int rows)
{
	long total = (long)rows * n;
	if (total <= 0) return;
	if (n >= ROWK && n % 4 == 0 && amode == 0 && bmode == 0 && al16(o, ors) && al16(a.p, a.rs) && al16(b.p, b.rs)) {
		const int cpr = (n + TPB * EPT * 4 - 1) / (TPB * EPT * 4);
		const unsigned grid = (unsigned)((long)rows * cpr);
		switch (op) {
#define BIN(K) \
	case K: binary_rows4_k<K><<<grid, TPB, 0, s>>>(o, ors, n, a, b, cpr); break;
			BIN(TGK_ADD) BIN(TGK_SUB) BIN(TGK_MUL) BIN(TGK_DIV) BIN(TGK_MAX) BIN(TGK_MIN)
#undef BIN
		default: break;
		}
	} else if (n >= ROWK) {
		const int cpr = (n + TPB * EPT - 1) / (TPB * EPT);
		const unsigned grid = (unsigned)((long)rows * cpr);
		switch (op) {
#define BIN(K) \
	case K: binary_rows_k<K><<<grid, TPB, 0, s>>>(o, ors, n, a, amode, amap, aper, b, bmode, bmap, bper, cpr); break;
			BIN(TGK_ADD) BIN(TGK_SUB) BIN(TGK_MUL) BIN(TGK_DIV) BIN(TGK_MAX) BIN(TGK_MIN)
#undef BIN
		default: break;
		}
	} else
		binary_k<<<blocks_for(total), TPB, 0, s>>>(op, o, ors, n, a, amode, amap, aper, b, bmode, bmap, bper, total);
}

void tgk_unary(hipStream_t s, int op, float *o, long ors, tgk_opd a, int n, int rows)
{
	long total = (long)rows * n;
	if (total <= 0) return;
	if (n >= ROWK && n % 4 == 0 && al16(o, ors) && al16(a.p, a.rs)) {
		const int cpr = (n + TPB * EPT * 4 - 1) / (TPB * EPT * 4);
		const unsigned grid = (unsigned)((long)rows * cpr);
		switch (op) {
#define UN(K) \
	case K: unary_rows4_k<K><<<grid, TPB, 0, s>>>(o, ors, a, n, cpr); break;
			UN(TGM_NEG) UN(TGM_TANH) UN(TGM_RELU) UN(TGM_SIGMOID) UN(TGM_EXP) UN(TGM_SQRT) UN(TGM_GELU) UN(TGM_SILU)
			UN(TGM_SOFTPLUS) UN(TGM_LOG) UN(TGM_SIN) UN(TGM_COS) UN(TGM_FLOOR) UN(TGM_STEP)
#undef UN
		default: break;
		}
	} else if (n >= ROWK) {
		const int cpr = (n + TPB * EPT - 1) / (TPB * EPT);
		const unsigned grid = (unsigned)((long)rows * cpr);
		switch (op) {
#define UN(K) \
	case K: unary_rows_k<K><<<grid, TPB, 0, s>>>(o, ors, a, n, cpr); break;
			UN(TGM_NEG) UN(TGM_TANH) UN(TGM_RELU) UN(TGM_SIGMOID) UN(TGM_EXP) UN(TGM_SQRT) UN(TGM_GELU) UN(TGM_SILU)
			UN(TGM_SOFTPLUS) UN(TGM_LOG) UN(TGM_SIN) UN(TGM_COS) UN(TGM_FLOOR) UN(TGM_STEP)
#undef UN
		default: break;
		}
	} else
		unary_k<<<blocks_for(total), TPB, 0, s>>>(op, o, ors, a, n, total);
}

void tgk_ew_run(hipStream_t s, const tgk_ew *e, int n, int rows)
{
	if (rows <= 0 || n <= 0 || e->nin < 1 || e->nin > TGK_EW_MAXIN) return;
	bool vec = n % 4 == 0;
	int n0 = 0; // leading inputs that load as float4
	while (n0 < e->nin && (e->in_mode[n0] == 0 || (e->in_mode[n0] == 3 && e->in_per[n0] % 4 == 0 && n / e->in_per[n0] < (1 << 22))))
		n0++;
	for (int j = 0; j < n0; j++) vec = vec && ((size_t)e->in[j] & 15) == 0 && e->in_rs[j] % 4 == 0;
	for (int j = 0; j < e->nout; j++) vec = vec && ((size_t)e->out[j] & 15) == 0 && e->out_rs[j] % 4 == 0;
	const int cpr = (n + TPB * 4 - 1) / (TPB * 4);
	const unsigned grid = (unsigned)((long)rows * cpr);
	if (!vec) {
		ew_k<0, false><<<grid, TPB, 0, s>>>(*e, n, cpr);
		return;
	}
	switch (n0) {
	case 0: ew_k<0, true><<<grid, TPB, 0, s>>>(*e, n, cpr); break;
	case 1: ew_k<1, true><<<grid, TPB, 0, s>>>(*e, n, cpr); break;
	case 2: ew_k<2, true><<<grid, TPB, 0, s>>>(*e, n, cpr); break;
	case 3: ew_k<3, true><<<grid, TPB, 0, s>>>(*e, n, cpr); break;
	case 4: ew_k<4, true><<<grid, TPB, 0, s>>>(*e, n, cpr); break;
	case 5: ew_k<5, true><<<grid, TPB, 0, s>>>(*e, n, cpr); break;
	default: ew_k<6, true><<<grid, TPB, 0, s>>>(*e, n, cpr); break;
	}
}

// f32 products (quant 0) in tiles: a block computes a TS x TS tile of one
// (batch row, group) product, each of its 16 x 16 threads a TS/16 x TS/16
// block of it. A and B pass through LDS 16 values of p at a time, and every
// output adds its products in order p = 0..kend-1 from 0.0f with separate
// multiply and add, exactly as mm_exact_k does, so the results are
// bit-identical to it. Tile rows, columns and p values past m, n and k read
// as zeros; the p loop stops at kend and nothing past m or n is stored.
template <int TS>
__device__ inline void mm_tile(const tgk_mm &d, const float *A, const float *B, float *O, int i0, int j0, int kend, float (*As)[TS + 4],
			       float (*Bs)[TS + 4])
{
	constexpr int KC = 16, R = TS / 16, NE = TS * KC / 256; // tile elements per thread and chunk
	const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
	float acc[R][R];
	for (int u = 0; u < R; u++)
		for (int v = 0; v < R; v++) acc[u][v] = 0.0f;
	// chunk p0's A and B elements of this thread into registers (the next
	// chunk's loads are in flight while the current one is multiplied)
	float ra[NE], rb[NE];
	auto fetch = [&](int p0) {
		for (int q = 0; q < NE; q++) { // A, coalesced along whichever of i, p is unit stride
			const int e = threadIdx.x + q * 256;
			int i, p;
			if (d.ap == 1) i = e / KC, p = e % KC;
			else p = e / TS, i = e % TS;
			const bool in = i0 + i < d.m && p0 + p < d.k;
			const float x = A[in ? (long)(i0 + i) * d.ai + (long)(p0 + p) * d.ap : 0];
			ra[q] = in ? x : 0.0f;
		}
		for (int q = 0; q < NE; q++) { // B
			const int e = threadIdx.x + q * 256;
			int j, p;
			if (d.bj == 1 || d.bp != 1) p = e / TS, j = e % TS;
			else j = e / KC, p = e % KC;
			const bool in = j0 + j < d.n && p0 + p < d.k;
			const float x = B[in ? (long)(p0 + p) * d.bp + (long)(j0 + j) * d.bj : 0];
			rb[q] = in ? x : 0.0f;
		}
	};
	auto stash = [&]() {
		for (int q = 0; q < NE; q++) {
			const int e = threadIdx.x + q * 256;
			if (d.ap == 1) As[e % KC][e / KC] = ra[q];
			else As[e / TS][e % TS] = ra[q];
			if (d.bj == 1 || d.bp != 1) Bs[e / TS][e % TS] = rb[q];
			else Bs[e % KC][e / KC] = rb[q];
		}
	};
	if (kend > 0) {
		fetch(0);
		stash();
	}
	__syncthreads();
	for (int p0 = 0; p0 < kend; p0 += KC) {
		const bool more = p0 + KC < kend;
		if (more) fetch(p0 + KC);
		const int kk = kend - p0 < KC ? kend - p0 : KC;
		for (int p = 0; p < kk; p++) {
			float a[R], b[R];
			for (int u = 0; u < R; u++) a[u] = As[p][ty * R + u];
			for (int v = 0; v < R; v++) b[v] = Bs[p][tx * R + v];
			for (int u = 0; u < R; u++)
				for (int v = 0; v < R; v++) acc[u][v] = acc[u][v] + a[u] * b[v];
		}
		__syncthreads();
		if (more) {
			stash();
			__syncthreads();
		}
	}
	for (int u = 0; u < R; u++) {
		const int i = i0 + ty * R + u;
		if (i >= d.m) break;
		for (int v = 0; v < R; v++) {
			const int j = j0 + tx * R + v;
			if (j < d.n) O[(long)i * d.oi + (long)j * d.oj] = acc[u][v];
		}
	}
}

// The grid: tm x tn tiles per (batch row, group). Causal products (square
// tiles, mode = d.causal as the launcher allows it): mode 1 enumerates only the tiles on or below the diagonal
// (tn counts them, ti >= tj, all of equal work); mode 2 gives a block the row
// tiles p and tm - 1 - p of one column tile (tm counts the pairs), whose sums
// run to the end of each tile's rows, so every block has the same work.
template <int TS>
__global__ __launch_bounds__(256) void mm_tile_k(tgk_mm d, int tm, int tn, int nt, int mode)
{
	__shared__ float As[16][TS + 4]; // As[p][i]
	__shared__ float Bs[16][TS + 4]; // Bs[p][j]
	const int tiles = tm * tn;
	const long rg = blockIdx.x / tiles;
	const int t = (int)(blockIdx.x - rg * tiles);
	const long r = rg / d.g;
	const int g = (int)(rg - r * d.g);
	const float *A = d.a.p + r * d.a.rs + g * d.ag, *B = d.b.p + r * d.b.rs + g * d.bg;
	float *O = d.o + r * d.ors + g * d.og;
	if (mode == 1) { // lower-triangle tile t: ti (ti + 1) / 2 <= t < (ti + 1) (ti + 2) / 2
		int ti = (int)((sqrtf(8.0f * t + 1.0f) - 1.0f) * 0.5f);
		while (ti * (ti + 1) / 2 > t) ti--;
		while ((ti + 1) * (ti + 2) / 2 <= t) ti++;
		const int tj = t - ti * (ti + 1) / 2;
		mm_tile<TS>(d, A, B, O, ti * TS, tj * TS, d.k, As, Bs);
	} else if (mode == 2) {
		const int pr = t / tn, tj = t - pr * tn;
		for (int h = 0; h < 2; h++) {
			const int ti = h == 0 ? pr : nt - 1 - pr;
			if (h == 1 && ti == pr) break; // the middle tile of an odd count
			const int i0 = ti * TS, kend = i0 + TS < d.k ? i0 + TS : d.k;
			mm_tile<TS>(d, A, B, O, i0, tj * TS, kend, As, Bs);
		}
	} else {
		const int ti = t / tn, tj = t - ti * tn;
		mm_tile<TS>(d, A, B, O, ti * TS, tj * TS, d.k, As, Bs);
	}
}

void tgk_matmul_exact(hipStream_t s, const tgk_mm *d, int rows)
{
	long total = (long)rows * d->g * d->m * d->n;
	if (total <= 0) return;
	if (d->quant == 0 && (long)d->m * d->n >= 64 * 64 && d->k >= 16) {
		const long rg = (long)rows * d->g;
		if (d->causal == 1 && d->m == d->n) { // 64 x 64 tiles on or below the diagonal
			const int nt = (d->m + 63) / 64, ntri = nt * (nt + 1) / 2;
			mm_tile_k<64><<<(unsigned)(rg * ntri), 256, 0, s>>>(*d, 1, ntri, nt, 1);
			return;
		}
		if (d->causal == 2) { // pairs of 64-row tiles
			const int nt = (d->m + 63) / 64, sn = (d->n + 63) / 64;
			mm_tile_k<64><<<(unsigned)(rg * ((nt + 1) / 2) * sn), 256, 0, s>>>(*d, (nt + 1) / 2, sn, nt, 2);
			return;
		}
		const int tm = (d->m + 127) / 128, tn = (d->n + 127) / 128;
		if (rg * tm * tn >= 1024) { // enough 128 x 128 tiles to fill the chip
			mm_tile_k<128><<<(unsigned)(rg * tm * tn), 256, 0, s>>>(*d, tm, tn, tm, 0);
		} else {
			const int sm = (d->m + 63) / 64, sn = (d->n + 63) / 64;
			mm_tile_k<64><<<(unsigned)(rg * sm * sn), 256, 0, s>>>(*d, sm, sn, sm, 0);
		}
		return;
	}
	mm_exact_k<<<blocks_for(total), TPB, 0, s>>>(*d, total);
}

void tgk_rowop(hipStream_t s, int op, float *o, long ors, tgk_opd a, int nrow, int cols, int rows)
{
	long total = (long)rows * nrow;
	if (total <= 0) return;
	if (a.rs == (long)nrow * cols && ors == (long)nrow * cols && total < (1L << 31)) {
		// rows back to back in memory on both sides: all lines of the pass are one row's lines
		// (lets one-line rows, such as one token each, share blocks)
		nrow = (int)total;
		rows = 1;
	}
	// lines 16-byte aligned and 4 banks apart when cols is a multiple of 4, else an odd stride
	const int stride = cols % 4 == 0 ? cols + 4 : cols | 1;
	// LDS: the lines and one value per line (padded to 4)
	auto lds_bytes = [&](long l) { return (l * stride + ((l + 3) & ~3L)) * 4; };
	int lpb = 32; // a power of two, so TPB / lpb threads share a line's max
	while (lpb > 1 && (lds_bytes(lpb) > 65536 || nrow % lpb)) lpb >>= 1;
	while (lpb > 4 && (long)rows * (nrow / lpb) < 512) lpb >>= 1; // few lines: spread them over more blocks
	if (cols >= 32 && lpb >= 4 && lds_bytes(lpb) <= 65536 && (long)rows * (nrow / lpb) < (1L << 31))
		rowop_lds_k<<<(unsigned)(rows * (long)(nrow / lpb)), TPB, (size_t)lds_bytes(lpb), s>>>(op, o, ors, a, nrow, cols, lpb, stride);
	else
		rowop_k<<<blocks_for(total), TPB, 0, s>>>(op, o, ors, a, nrow, cols, total);
}

namespace {
// every 16-byte word of the span once, grid-stride; a lane writes only when
// its sum has a value that no input of the benchmark produces (never), so
// the loads cannot be dropped
typedef int rd_v4i __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void read_k(const rd_v4i *p, long n16, int *sink)
{
	const long t = (long)blockIdx.x * 256 + threadIdx.x, nt = (long)gridDim.x * 256;
	int acc = 0;
	for (long i = t; i < n16; i += nt) {
		const rd_v4i v = __builtin_nontemporal_load(p + i);
		acc ^= v.x ^ v.y ^ v.z ^ v.w;
	}
	if (acc == 0x7fa55a5f) sink[0] = acc;
}
} // namespace

void tgk_read(hipStream_t s, const void *p, size_t bytes, int blocks, int *sink)
{
	if (bytes >= 16 && blocks > 0) read_k<<<(unsigned)blocks, 256, 0, s>>>((const rd_v4i *)p, (long)(bytes / 16), sink);
}

void tgk_reduce(hipStream_t s, int op, float *o, long ors, tgk_opd a, int n, int rows)
{
	// one wave per block while that leaves fewer than 1024 blocks: long rows
	// then spread over more compute units (each thread's adds are sequential)
	const int tpb = rows < 1024 * 64 ? 64 : TPB;
	if (rows > 0) reduce_k<<<(unsigned)((rows + tpb - 1) / tpb), tpb, 0, s>>>(op, o, ors, a, n, rows);
}

void tgk_transpose(hipStream_t s, float *o, long ors, tgk_opd a, int g, int r, int c, int rows)
{
	long total = (long)rows * g * r * c;
	if (total > 0) transpose_k<<<blocks_for(total), TPB, 0, s>>>(o, ors, a, g, r, c, total);
}

void tgk_outer(hipStream_t s, float *o, long ors, tgk_opd a, int m, tgk_opd b, int n, int rows)
{
	long total = (long)rows * m * n;
	if (total > 0) outer_k<<<blocks_for(total), TPB, 0, s>>>(o, ors, a, m, b, n, total);
}

void tgk_take(hipStream_t s, float *o, long ors, tgk_opd w, tgk_opd idx, int cnt, int d, int h, int rows)
{
	long total = (long)rows * cnt * h;
	if (total > 0) take_k<<<blocks_for(total), TPB, 0, s>>>(o, ors, w, idx, cnt, d, h, total);
}

void tgk_copy(hipStream_t s, float *o, long ors, long ooff, tgk_opd a, long aoff, int w, int rows)
{
	long total = (long)rows * w;
	if (total > 0) copy_k<<<blocks_for(total), TPB, 0, s>>>(o, ors, ooff, a, aoff, w, total);
}

namespace {

// The selective-scan recurrence of a Mamba-style block (the scan body
//   dA = exp(reshape(dt_t) * A); h = dA * h + outer(du_t, B_t); y_t = h @ C_t
// recognized by the program builder), fused over all T steps: one thread
// per (row, channel d) keeps h[d, 0..N-1] and A[d, :] in registers. Each
// product, exponential and sum is the one the per-instruction kernels compute
// (binary_k, unary_k, outer_k, mm_exact_k; this file is built with
// -ffp-contract=off), in the same order, so the results are bit-identical to
// running the body one instruction per launch. A block covers channels of
// a single row, so B_t and C_t are the same for every lane of a wave.
// DUX: du_t = dt_t * dux_t, formed as the steps are loaded (the instruction
// that made the du sequence, folded in). GATE: the stacked output is
// (y_t + gx_t * gD) * silu(gz_t) (Mamba's gate, the four instructions after
// the scan, folded in), each operation as the elementwise kernels compute it
// (tg_ewop.h); a chunk's gate operands are loaded as the chunk starts and its
// outputs gated once its steps are done.
template <int N, bool DUX, bool GATE>
__global__ __launch_bounds__(256) void sscan_k(float *h, long hrs, tgk_opd dt, tgk_opd du, tgk_opd Bq, tgk_opd Cq, tgk_opd A,
					       float *ys, long yrs, int D, int T, int reverse, int dblocks, tgk_sscan_fuse fu)
{
	// Steps go in chunks of U. While chunk c is computed, chunk c + 1's dt and
	// du are in flight into registers and its B and C into registers bound
	// for the other LDS buffer, so the step loop never waits on memory.
	// (8 steps a chunk with the gate folded in: its operands and outputs are
	// buffered per chunk, and the registers decide how many waves share a SIMD)
	constexpr int U = GATE ? 8 : 16, BC = U * 2 * N, PER = (BC + 255) / 256;
	__shared__ float bc[2][BC]; // [step][B_0 .. B_N-1, C_0 .. C_N-1]
	const int r = blockIdx.x / dblocks;
	const int d = (blockIdx.x - r * dblocks) * 256 + threadIdx.x;
	const bool live = d < D;
	const int dd = live ? d : D - 1; // lanes past D shadow channel D - 1 and store nothing
	float hv[N], av[N];
	float *hp = h + (long)r * hrs + (long)dd * N;
	for (int n = 0; n < N; n++) {
		hv[n] = hp[n];
		av[n] = A.p[(long)r * A.rs + (long)dd * N + n];
	}
	const float *dtp = dt.p + (long)r * dt.rs, *dup = (DUX ? fu.dux : du).p + (long)r * (DUX ? fu.dux : du).rs;
	const float *bp = Bq.p + (long)r * Bq.rs, *cp = Cq.p + (long)r * Cq.rs;
	float *yp = ys + (long)r * yrs;
	auto tstep = [&](int s) { return reverse ? T - 1 - s : s; };
	auto load_dd = [&](int s0, float *a, float *b) {
		for (int u = 0; u < U; u++) {
			const int t = tstep(s0 + u < T ? s0 + u : T - 1);
			a[u] = dtp[(long)t * D + dd];
			b[u] = dup[(long)t * D + dd];
		}
		if constexpr (DUX)
			for (int u = 0; u < U; u++) b[u] = tg_bop(TGK_MUL, a[u], b[u]);
	};
	const float *gxp = GATE ? fu.gx.p + (long)r * fu.gx.rs : nullptr, *gzp = GATE ? fu.gz.p + (long)r * fu.gz.rs : nullptr;
	const float gdv = GATE ? fu.gD[dd] : 0.0f;
	float gxc[GATE ? U : 1], gzc[GATE ? U : 1], yb[GATE ? U : 1];
	float bcr[PER];
	auto load_bc = [&](int s0) {
		for (int j = 0; j < PER; j++) {
			const int e = (int)threadIdx.x + j * 256, ec = e < BC ? e : BC - 1;
			const int u = ec / (2 * N), q = ec - u * (2 * N);
			const int t = tstep(s0 + u < T ? s0 + u : T - 1);
			bcr[j] = q < N ? bp[(long)t * N + q] : cp[(long)t * N + q - N];
		}
	};
	auto store_bc = [&](int buf) {
		for (int j = 0; j < PER; j++) {
			const int e = (int)threadIdx.x + j * 256;
			if (e < BC) bc[buf][e] = bcr[j];
		}
	};
	float dtc[U], duc[U], dtn[U], dun[U];
	load_dd(0, dtc, duc);
	load_bc(0);
	store_bc(0);
	__syncthreads();
	for (int s0 = 0, c = 0; s0 < T; s0 += U, c++) {
		const bool more = s0 + U < T;
		if (more) {
			load_dd(s0 + U, dtn, dun);
			load_bc(s0 + U);
		}
		const float *bcb = bc[c & 1];
		float *yt = yp + (long)tstep(s0) * D + d;
		const long ystep = reverse ? -(long)D : (long)D;
		if constexpr (GATE)
			for (int u = 0; u < U; u++) {
				const long t = tstep(s0 + u < T ? s0 + u : T - 1);
				gxc[u] = gxp[t * D + dd];
				gzc[u] = gzp[t * D + dd];
			}
#pragma unroll
		for (int u = 0; u < U; u++) {
			if (s0 + u < T) {
				float y = 0.0f;
#pragma unroll
				for (int n = 0; n < N; n++) {
					const float da = expf(dtc[u] * av[n]);
					const float hn = da * hv[n] + duc[u] * bcb[u * 2 * N + n];
					hv[n] = hn;
					y = y + hn * bcb[u * 2 * N + N + n];
				}
				if constexpr (GATE) yb[u] = y;
				else if (live) yt[u * ystep] = y;
			}
		}
		if constexpr (GATE)
			for (int u = 0; u < U; u++)
				if (s0 + u < T && live)
					yt[u * ystep] = tg_bop(TGK_MUL, tg_bop(TGK_ADD, yb[u], tg_bop(TGK_MUL, gxc[u], gdv)), tg_uop(TGM_SILU, gzc[u]));
		if (more) {
			store_bc((c + 1) & 1);
			for (int u = 0; u < U; u++) dtc[u] = dtn[u], duc[u] = dun[u];
		}
		__syncthreads();
	}
	if (live)
		for (int n = 0; n < N; n++) hp[n] = hv[n];
}

} // namespace

bool tgk_sscan_supported(int N) { return N == 4 || N == 8 || N == 16; }

namespace {

template <int N>
void launch_sscan(hipStream_t s, unsigned grid, float *h, long hrs, tgk_opd dt, tgk_opd du, tgk_opd Bq, tgk_opd Cq, tgk_opd A, float *ys,
		  long yrs, int D, int T, int reverse, int dblocks, const tgk_sscan_fuse &f)
{
	const bool dux = f.dux.p != nullptr, gate = f.gx.p != nullptr;
	if (dux && gate) sscan_k<N, true, true><<<grid, 256, 0, s>>>(h, hrs, dt, du, Bq, Cq, A, ys, yrs, D, T, reverse, dblocks, f);
	else if (dux) sscan_k<N, true, false><<<grid, 256, 0, s>>>(h, hrs, dt, du, Bq, Cq, A, ys, yrs, D, T, reverse, dblocks, f);
	else if (gate) sscan_k<N, false, true><<<grid, 256, 0, s>>>(h, hrs, dt, du, Bq, Cq, A, ys, yrs, D, T, reverse, dblocks, f);
	else sscan_k<N, false, false><<<grid, 256, 0, s>>>(h, hrs, dt, du, Bq, Cq, A, ys, yrs, D, T, reverse, dblocks, f);
}

} // namespace

void tgk_sscan(hipStream_t s, float *h, long hrs, tgk_opd dt, tgk_opd du, tgk_opd Bq, tgk_opd Cq, tgk_opd A, float *ys, long yrs, int D,
	       int N, int T, int reverse, int rows, const tgk_sscan_fuse *fuse)
{
	if (rows <= 0 || D <= 0 || T <= 0) return; // T = 0: the carry keeps its initial value
	const int dblocks = (D + 255) / 256;
	const unsigned grid = (unsigned)(rows * dblocks);
	const tgk_sscan_fuse f = fuse ? *fuse : tgk_sscan_fuse{};
	switch (N) {
	case 4: launch_sscan<4>(s, grid, h, hrs, dt, du, Bq, Cq, A, ys, yrs, D, T, reverse, dblocks, f); break;
	case 8: launch_sscan<8>(s, grid, h, hrs, dt, du, Bq, Cq, A, ys, yrs, D, T, reverse, dblocks, f); break;
	case 16: launch_sscan<16>(s, grid, h, hrs, dt, du, Bq, Cq, A, ys, yrs, D, T, reverse, dblocks, f); break;
	default: break;
	}
}
