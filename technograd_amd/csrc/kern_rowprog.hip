// Row-program interpreter: one lane runs one batch row through the whole
// model, so per-row control flow (think loops with data-dependent halting,
// scans) needs no host round trips and no masks: a lane whose row has halted
// simply leaves the loop. Values of all lanes live in one device arena laid
// out [slot][lane] (structure of arrays), so the lanes of a wave touch
// consecutive words; params and constants are read from a shared pool with
// wave-uniform addresses.
//
// Two number systems share the interpreter:
//   f32      the reference interpreter's kernels (runtime/tg_rt.h): sums in
//            index order from 0.0f, separate multiply and add
//            (-ffp-contract=off), correctly rounded division and sqrt;
//   Q16.16   the fixed-point kernels (runtime/tg_rtq.h) in the instruction
//            order of a `tgc c --fixed` unit (src/cgen.c:100-314): int64
//            accumulation rounded once, saturation, Q7.24 quant scales.
// Q16.16 results are bit-exact with the reference, including its tg_fdiv
// rounding for negative divisors (the half-divisor is added on the side that
// makes the quotient's magnitude one smaller for most inputs).
#include "tg_devmath.h"
#include "tg_kern.h"
#include "tg_rowdev.h"
#include "tgm.h"

#include <climits>
#include <math.h>

namespace {

constexpr int MAXF = 8; // nested loop frames

using namespace tgrd;

__device__ inline int unq(int op, int x)
{
	switch (op) {
	case TGM_NEG: return negq(x);
	case TGM_TANH: return tanhq(x);
	case TGM_RELU: return reluq(x);
	case TGM_SIGMOID: return sigmoidq(x);
	case TGM_EXP: return expq(x);
	case TGM_SQRT: return sqrtq(x);
	case TGM_GELU: return geluq(x);
	case TGM_SILU: return siluq(x);
	case TGM_SOFTPLUS: return softplusq(x);
	case TGM_LOG: return logq(x);
	case TGM_SIN: return sinq(x);
	case TGM_COS: return cosq(x);
	case TGM_FLOOR: return floorq(x);
	default: return stepq(x);
	}
}

__device__ inline int binq(int op, int x, int y)
{
	switch (op) {
	case TGK_ADD: return addq(x, y);
	case TGK_SUB: return subq(x, y);
	case TGK_MUL: return fmulq(x, y);
	case TGK_DIV: return fdivq(x, y);
	case TGK_MAX: return maxq(x, y);
	default: return minq(x, y);
	}
}

__device__ inline float binf(int op, float x, float y)
{
	switch (op) {
	case TGK_ADD: return x + y;
	case TGK_SUB: return x - y;
	case TGK_MUL: return x * y;
	case TGK_DIV: return x / y;
	case TGK_MAX: return maxf_(x, y);
	default: return minf_(x, y);
	}
}

__device__ inline float unf(int op, float x)
{
	switch (op) {
	case TGM_NEG: return negf_(x);
	case TGM_TANH: return tanhf(x);
	case TGM_RELU: return reluf_(x);
	case TGM_SIGMOID: return sigmoidf_(x);
	case TGM_EXP: return expf(x);
	case TGM_SQRT: return sqrtf(x);
	case TGM_GELU: return geluf_(x);
	case TGM_SILU: return siluf_(x);
	case TGM_SOFTPLUS: return softplusf_(x);
	case TGM_LOG: return logf(x);
	case TGM_SIN: return sinf(x);
	case TGM_COS: return cosf(x);
	case TGM_FLOOR: return floorf(x);
	default: return stepf_(x);
	}
}

// An operand view for one lane: element i at base[i * st].
struct View {
	float *base;
	long st;
	__device__ inline float &f(long i) const { return base[i * st]; }
	__device__ inline int &q(long i) const { return reinterpret_cast<int *>(base)[i * st]; }
};

struct Frame {
	int pc0, it, lim, t, sv;
	float svf;
};

template <bool FX>
__global__ __launch_bounds__(256) void rowprog_k(rp_args A)
{
	long row = (long)blockIdx.x * blockDim.x + threadIdx.x;
	if (row >= A.rows) return;
	const long R = A.R;
	float *ar = A.arena + row;
	auto view = [&](int ref) -> View {
		if (ref >= 0) return View{ ar + (long)ref * R, R };
		return View{ const_cast<float *>(A.pool) + (-(long)ref - 1), 1 };
	};
	for (int i = 0; i < A.per; i++) ar[(long)(A.in_slot + i) * R] = A.in[row * A.per + i];
	Frame fr[MAXF];
	int nf = 0;
	for (int pc = 0; pc < A.nins;) {
		const rp_ins I = A.prog[pc];
		View o = view(I.out), a = view(I.a), b = view(I.b);
		switch (I.kind) {
		case RP_BIN: {
			const int *am = A.imap + I.p[1], *bm = A.imap + I.p[3];
			for (int i = 0; i < I.n; i++) {
				long ia = I.p[0] == 0 ? i : I.p[0] == 1 ? 0 : am[i], ib = I.p[2] == 0 ? i : I.p[2] == 1 ? 0 : bm[i];
				if (FX) o.q(i) = binq(I.op, a.q(ia), b.q(ib));
				else o.f(i) = binf(I.op, a.f(ia), b.f(ib));
			}
			break;
		}
		case RP_UN:
			for (int i = 0; i < I.n; i++) {
				if (FX) o.q(i) = unq(I.op, a.q(i));
				else o.f(i) = unf(I.op, a.f(i));
			}
			break;
		case RP_MM: {
			const int G = I.p[0], M = I.p[1], K = I.p[2], N = I.p[3], quant = I.p[4], bits = I.p[5];
			const uint8_t *codes = A.codes + I.p[6];
			if (!FX && I.p[8] && G == 1) { /* calibration: this product's samples, as the reference's hook sees them */
				const int c = I.p[8] - 1, add = I.p[9] ? M : N;
				int *cnt = A.cap_count + (long)c * A.rows + row;
				if (*cnt + add <= A.cap_rows[c]) {
					float *dst = A.cap + A.cap_base[c] + ((long)row * A.cap_rows[c] + *cnt) * K;
					if (I.p[9])
						for (int i = 0; i < M; i++)
							for (int r = 0; r < K; r++) dst[(long)i * K + r] = a.f((long)i * K + r);
					else
						for (int j = 0; j < N; j++)
							for (int r = 0; r < K; r++) dst[(long)j * K + r] = b.f((long)r * N + j);
				}
				*cnt += add;
			}
			for (int g = 0; g < G; g++)
				for (int i = 0; i < M; i++)
					for (int j = 0; j < N; j++) {
						long ai = (long)g * M * K + (long)i * K, bj = (long)g * K * N + j, oi = (long)g * M * N + (long)i * N + j;
						if (FX) {
							long s = 0;
							if (quant == 1) {
								for (int p = 0; p < K; p++) s += (long)qcode(codes, bits, (long)i * K + p) * b.q(bj + (long)p * N);
								o.q(oi) = qscaleq(s, A.qscale[I.p[7] + i]);
							} else if (quant == 2) {
								for (int p = 0; p < K; p++) s += (long)a.q(ai + p) * qcode(codes, bits, (long)p * N + j);
								o.q(oi) = qscaleq(s, A.qscale[I.p[7] + j]);
							} else {
								for (int p = 0; p < K; p++) s += (long)a.q(ai + p) * b.q(bj + (long)p * N);
								o.q(oi) = sat((s + 32768) >> 16);
							}
						} else {
							float s = 0.0f;
							if (quant == 1) {
								for (int p = 0; p < K; p++) s += (float)qcode(codes, bits, (long)i * K + p) * b.f(bj + (long)p * N);
								s = A.fscale[I.p[7] + i] * s;
							} else if (quant == 2) {
								for (int p = 0; p < K; p++) s += a.f(ai + p) * (float)qcode(codes, bits, (long)p * N + j);
								s = A.fscale[I.p[7] + j] * s;
							} else {
								for (int p = 0; p < K; p++) s += a.f(ai + p) * b.f(bj + (long)p * N);
							}
							o.f(oi) = s;
						}
					}
			break;
		}
		case RP_ROW: {
			const int nrow = I.p[0], cols = I.p[1];
			for (int q = 0; q < nrow; q++) {
				long base = (long)q * cols;
				if (FX) {
					if (I.op == TGM_SOFTMAX) {
						int mx = a.q(base);
						long s = 0;
						for (int i = 1; i < cols; i++) mx = a.q(base + i) > mx ? a.q(base + i) : mx;
						for (int i = 0; i < cols; i++) {
							o.q(base + i) = expq_neg(subq(a.q(base + i), mx)); // x - max <= 0
							s += o.q(base + i);
						}
						for (int i = 0; i < cols; i++) o.q(base + i) = softq(o.q(base + i), s);
					} else {
						unsigned long ss = 0;
						for (int i = 0; i < cols; i++) ss += (unsigned long)((long)a.q(base + i) * a.q(base + i));
						const int rms = rmsq(ss, cols);
						for (int i = 0; i < cols; i++) o.q(base + i) = fdivq(a.q(base + i), rms);
					}
				} else {
					if (I.op == TGM_SOFTMAX) {
						float mx = a.f(base), s = 0.0f;
						for (int i = 1; i < cols; i++)
							if (a.f(base + i) > mx) mx = a.f(base + i);
						for (int i = 0; i < cols; i++) {
							o.f(base + i) = expf(a.f(base + i) - mx);
							s += o.f(base + i);
						}
						for (int i = 0; i < cols; i++) o.f(base + i) /= s;
					} else {
						float s = 0.0f;
						for (int i = 0; i < cols; i++) s += a.f(base + i) * a.f(base + i);
						float inv = 1.0f / sqrtf(s / (float)cols + 1e-6f);
						for (int i = 0; i < cols; i++) o.f(base + i) = a.f(base + i) * inv;
					}
				}
			}
			break;
		}
		case RP_RED:
			if (FX) {
				long s = 0;
				for (int i = 0; i < I.n; i++) s += a.q(i);
				o.q(0) = I.op == TGM_SUM ? sat(s) : sat(s / I.n);
			} else {
				float s = 0.0f;
				for (int i = 0; i < I.n; i++) s += a.f(i);
				o.f(0) = I.op == TGM_SUM ? s : s / (float)I.n;
			}
			break;
		case RP_TRANS: {
			const int G = I.p[0], RR = I.p[1], C = I.p[2];
			for (int z = 0; z < G; z++)
				for (int i = 0; i < RR; i++)
					for (int j = 0; j < C; j++) o.f((long)z * RR * C + (long)j * RR + i) = a.f((long)z * RR * C + (long)i * C + j);
			break;
		}
		case RP_OUTER:
			for (int i = 0; i < I.p[0]; i++)
				for (int j = 0; j < I.p[1]; j++) {
					long e = (long)i * I.p[1] + j;
					if (FX) o.q(e) = fmulq(a.q(i), b.q(j));
					else o.f(e) = a.f(i) * b.f(j);
				}
			break;
		case RP_COPY: {
			long ooff = I.p[0], aoff = I.p[1];
			if (I.p[2]) aoff += (long)fr[nf - 1].t * I.n;
			if (I.p[3]) ooff += (long)fr[nf - 1].t * I.n;
			for (int i = 0; i < I.n; i++) o.f(ooff + i) = a.f(aoff + i);
			break;
		}
		case RP_TAKE: {
			const int cnt = I.p[0], d = I.p[1], h = I.p[2];
			for (int i = 0; i < cnt; i++) {
				int t;
				if (FX) {
					long rr = ((long)b.q(i) + 32768) >> 16;
					t = rr >= 0 && rr < d ? (int)rr : -1;
				} else {
					float rr = floorf(b.f(i) + 0.5f);
					t = rr >= 0.0f && rr < (float)d ? (int)rr : -1;
				}
				for (int j = 0; j < h; j++) o.f((long)i * h + j) = t >= 0 ? a.f((long)t * h + j) : (FX ? 0.0f : 0.0f);
			}
			break;
		}
		case RP_THINK: {
			for (int i = 0; i < I.n; i++) o.f(i) = a.f(i);
			fr[nf].pc0 = pc + 1;
			fr[nf].it = 0;
			fr[nf].sv = ONE;
			fr[nf].svf = 1.0f;
			nf++;
			pc++;
			continue;
		}
		case RP_THINK_END: {
			const rp_ins T = A.prog[I.p[0]];
			Frame &f = fr[nf - 1];
			View st = view(T.out), y = view(T.p[0]);
			f.it++;
			bool stop = false;
			if (FX) {
				int d = 0;
				for (int i = 0; i < T.n; i++) {
					int e = absq(sat((long)y.q(i) - st.q(i)));
					d = e > d ? e : d;
				}
				for (int i = 0; i < T.n; i++) st.q(i) = y.q(i);
				if (T.p[2] >= 0 && d <= T.p[7]) stop = true;
				if (!stop && T.p[3] != INT_MIN) {
					int h = view(T.p[3]).q(0), p = h < 0 ? 0 : h > ONE ? ONE : h;
					f.sv = fmulq(f.sv, ONE - p);
					if (ONE - f.sv > T.p[8]) stop = true;
				}
			} else {
				float d = 0.0f;
				for (int i = 0; i < T.n; i++) {
					float e = fabsf(y.f(i) - st.f(i));
					if (e > d) d = e;
				}
				for (int i = 0; i < T.n; i++) st.f(i) = y.f(i);
				float eps = __int_as_float(T.p[2]);
				if (eps >= 0.0f && d <= eps) stop = true;
				if (!stop && T.p[3] != INT_MIN) {
					float p = view(T.p[3]).f(0);
					f.svf *= 1.0f - (p < 0.0f ? 0.0f : p > 1.0f ? 1.0f : p);
					if (1.0f - f.svf > __int_as_float(T.p[4])) stop = true;
				}
			}
			if (stop || f.it >= T.p[1]) {
				A.steps[row * A.nthink + T.p[5]] = f.it;
				nf--;
				pc++;
			} else {
				pc = f.pc0;
			}
			continue;
		}
		case RP_SCAN:
			fr[nf].pc0 = pc + 1;
			fr[nf].it = 0;
			fr[nf].lim = I.p[0];
			fr[nf].t = I.p[1] ? I.p[0] - 1 : 0;
			nf++;
			pc++;
			continue;
		case RP_SCAN_END: {
			const rp_ins S = A.prog[I.p[0]];
			Frame &f = fr[nf - 1];
			f.it++;
			if (f.it >= f.lim) {
				if (S.p[2] >= 0) A.steps[row * A.nthink + S.p[2]] = f.lim;
				nf--;
				pc++;
			} else {
				f.t = S.p[1] ? f.lim - 1 - f.it : f.it;
				pc = f.pc0;
			}
			continue;
		}
		default: break;
		}
		pc++;
	}
	View res = view(A.out_ref);
	for (int i = 0; i < A.nout; i++) A.out[row * A.nout + i] = res.f(i);
}

// H[r][c] = sum of x_r x_c over the samples, rows in order and each row's
// samples in the order its products ran, skipping x_r == 0: the additions of
// src/quant.c:100-115 in their order (each f64 product of two f32 is exact),
// so H is the reference's to the bit. Both triangles are summed (the skip
// makes H[r][c] and H[c][r] differ where an x is infinite).
__global__ __launch_bounds__(256) void hessian_k(const float *cap, const int *count, long row_cap, int K, int rows, double *H)
{
	const int c = blockIdx.x * 256 + threadIdx.x, r = blockIdx.y;
	if (c >= K) return;
	double s = 0.0;
	for (int row = 0; row < rows; row++) {
		const float *x = cap + (long)row * row_cap * K;
		const int n = count[row] < row_cap ? count[row] : (int)row_cap;
		for (int t = 0; t < n; t++) {
			const double xr = x[(long)t * K + r];
			if (xr != 0.0) s = s + xr * (double)x[(long)t * K + c];
		}
	}
	H[(long)r * K + c] = s;
}

} // namespace

void tgk_hessian(hipStream_t s, const float *cap, const int *count, long row_cap, int K, int rows, double *H)
{
	if (K <= 0) return;
	hessian_k<<<dim3((unsigned)((K + 255) / 256), (unsigned)K), 256, 0, s>>>(cap, count, row_cap, K, rows, H);
}

void tgk_rowprog(hipStream_t s, const rp_args *a)
{
	if (a->rows <= 0) return;
	unsigned blocks = (unsigned)((a->rows + 255) / 256);
	if (a->fixed) rowprog_k<true><<<blocks, 256, 0, s>>>(*a);
	else rowprog_k<false><<<blocks, 256, 0, s>>>(*a);
}
