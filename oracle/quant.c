/* TEST INFRASTRUCTURE ONLY — oracle post-training quantizer.
 *
 * Restates `tgc quantize` (src/quant.c):
 *   eligibility            use_axis/eligible  (quant.c:42-89)
 *   calibration Hessians   hook/calibrate     (quant.c:92-157), H = sum x x^T in double
 *   code rounding          code_of            (quant.c:176-181), nearbyint = ties to even
 *   clip search            best_scale         (quant.c:184-200), 10 candidates 1.0 .. 0.55
 *   Cholesky / inverse     cholesky, inv_chol_upper (quant.c:203-253)
 *   GPTQ error push        quantize_param     (quant.c:258-316), 1% dampening
 *   driver                 quantize_main      (quant.c:318-384): K > 2048 => no Hessian => RTN
 * The double-precision loops keep the reference's evaluation order, so codes
 * and scales are bit-identical.
 *
 * Pinned by: tests/golden/quant_* (codes and scales written by the reference's
 * own quantizer, built from its sources by oracle/Makefile, for int8 and int4,
 * both axes, RTN and GPTQ with text calibration rows): byte-identical TGIR. */
#include "tgo.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
	int v, axis, C, K;
	double *H;
	long nsamp;
} QP;

typedef struct {
	QP *p;
	int n;
} QSet;

static int use_axis(const tgo_module *m, int v, const tgo_block *b, int *axis)
{
	for (int i = 0; i < b->len; i++) {
		const tgo_ins *in = &b->v[i];
		if (in->op == O_THINK) {
			if (in->init == v || in->yield == v || !use_axis(m, v, in->body, axis)) return 0;
		} else if (in->op == O_SCAN) {
			for (int k = 0; k < in->nc; k++)
				if (in->cinit[k] == v || in->cnext[k] == v) return 0;
			for (int j = 0; j < in->nx; j++)
				if (in->x[j] == v) return 0;
			for (int y = 0; y < in->ny; y++)
				if (in->y[y] == v) return 0;
			if (!use_axis(m, v, in->body, axis)) return 0;
		} else {
			for (int j = 0; j < in->na; j++) {
				if (in->a[j] != v) continue;
				int a = tgo_q_axis_for(m, v, in);
				if (a < 0 || (*axis >= 0 && *axis != a)) return 0;
				*axis = a;
			}
		}
	}
	return 1;
}

static QSet eligible(const tgo_module *m, int min_size)
{
	QSet s = { NULL, 0 };
	for (int v = 0; v < m->nval; v++) {
		const tgo_value *x = &m->val[v];
		if (x->kind != TGO_PARAM || x->qbits || x->sh.rank != 2 || x->n < min_size) continue;
		if (x->name && !strncmp(x->name, "__", 2)) continue;
		if (m->output == v) continue;
		int axis = -1, ok = use_axis(m, v, &m->top, &axis);
		if (!ok || axis < 0) continue;
		s.p = realloc(s.p, (size_t)(s.n + 1) * sizeof *s.p);
		QP *q = &s.p[s.n++];
		memset(q, 0, sizeof *q);
		q->v = v;
		q->axis = axis;
		q->C = x->sh.dim[axis];
		q->K = x->sh.dim[1 - axis];
	}
	return s;
}

static void hook(void *ctx, const tgo_module *m, const tgo_ins *in, const float *a, const float *b)
{
	QSet *s = ctx;
	int mm, kk, nn, gg;
	tgo_matmul_dims(&m->val[in->a[0]].sh, &m->val[in->a[1]].sh, &mm, &kk, &nn, &gg);
	for (int i = 0; i < s->n; i++) {
		QP *q = &s->p[i];
		if (!q->H) continue;
		if (in->a[0] == q->v && q->axis == 0) {
			for (int j = 0; j < nn; j++, q->nsamp++)
				for (int r = 0; r < kk; r++) {
					double xr = b[r * nn + j];
					if (xr == 0) continue;
					for (int c = 0; c < kk; c++) q->H[r * kk + c] += xr * b[c * nn + j];
				}
		} else if (in->a[1] == q->v && q->axis == 1) {
			for (int r0 = 0; r0 < mm; r0++, q->nsamp++) {
				const float *x = a + (size_t)r0 * (size_t)kk;
				for (int r = 0; r < kk; r++) {
					double xr = x[r];
					if (xr == 0) continue;
					for (int c = 0; c < kk; c++) q->H[r * kk + c] += xr * x[c];
				}
			}
		}
	}
}

static void set_code(tgo_value *x, const QP *q, int c, int j, int code)
{
	long i = q->axis == 0 ? (long)c * q->K + j : (long)j * q->C + c;
	if (x->qbits == 8) {
		x->q[i] = (signed char)code;
		return;
	}
	unsigned char b = (unsigned char)x->q[i / 2];
	b = i % 2 ? (unsigned char)((b & 0x0f) | (unsigned char)((unsigned)code << 4)) : (unsigned char)((b & 0xf0) | (code & 0x0f));
	x->q[i / 2] = (signed char)b;
}

static int code_of(double w, double s, int lim)
{
	if (s <= 0) return 0;
	double r = nearbyint(w / s);
	return (int)(r > lim ? lim : r < -lim ? -lim : r);
}

static double best_scale(const double *w, int K, const double *hd, int lim)
{
	double amax = 0;
	for (int j = 0; j < K; j++)
		if (fabs(w[j]) > amax) amax = fabs(w[j]);
	if (amax == 0) return 1e-8;
	double best = INFINITY, bs = amax / lim;
	for (int g = 0; g < 10; g++) {
		double s = amax * (1.0 - 0.05 * g) / lim, e = 0;
		for (int j = 0; j < K; j++) {
			double d = w[j] - s * code_of(w[j], s, lim);
			e += d * d * (hd ? hd[j] : 1.0);
		}
		if (e < best) {
			best = e;
			bs = s;
		}
	}
	return bs;
}

static int cholesky(double *A, int n)
{
	for (int j = 0; j < n; j++) {
		double d = A[j * n + j];
		for (int k = 0; k < j; k++) d -= A[j * n + k] * A[j * n + k];
		if (d <= 0) return 0;
		d = sqrt(d);
		A[j * n + j] = d;
		for (int i = j + 1; i < n; i++) {
			double s = A[i * n + j];
			for (int k = 0; k < j; k++) s -= A[i * n + k] * A[j * n + k];
			A[i * n + j] = s / d;
		}
		for (int k = j + 1; k < n; k++) A[j * n + k] = 0;
	}
	return 1;
}

static int inv_chol_upper(const double *H, int n, double *U)
{
	double *L = malloc((size_t)n * (size_t)n * sizeof *L), *Li = malloc((size_t)n * (size_t)n * sizeof *Li);
	memcpy(L, H, (size_t)n * (size_t)n * sizeof *L);
	int ok = cholesky(L, n);
	if (ok) {
		for (long i = 0; i < (long)n * n; i++) Li[i] = 0;
		for (int c = 0; c < n; c++)
			for (int i = c; i < n; i++) {
				double s = i == c ? 1.0 : 0.0;
				for (int k = c; k < i; k++) s -= L[i * n + k] * Li[k * n + c];
				Li[i * n + c] = s / L[i * n + i];
			}
		for (int i = 0; i < n; i++)
			for (int j = i; j < n; j++) {
				double s = 0;
				for (int k = j; k < n; k++) s += Li[k * n + i] * Li[k * n + j];
				U[i * n + j] = U[j * n + i] = s;
			}
		ok = cholesky(U, n);
		if (ok)
			for (int i = 0; i < n; i++)
				for (int j = i + 1; j < n; j++) {
					U[i * n + j] = U[j * n + i];
					U[j * n + i] = 0;
				}
	}
	free(L);
	free(Li);
	return ok;
}

static void quantize_param(tgo_module *m, QP *q, int bits, int gptq, char *log, int logn)
{
	tgo_value *x = &m->val[q->v];
	int lim = bits == 8 ? 127 : 7, C = q->C, K = q->K;
	long n = (long)C * K;
	x->qbits = bits;
	x->qaxis = q->axis;
	x->q = calloc((size_t)(bits == 8 ? n : (n + 1) / 2), 1);
	x->qs = calloc((size_t)C, sizeof(float));
	double *W = malloc((size_t)n * sizeof *W), *hd = NULL, *U = NULL;
	for (int c = 0; c < C; c++)
		for (int j = 0; j < K; j++) W[(long)c * K + j] = q->axis == 0 ? x->data[(long)c * K + j] : x->data[(long)j * C + c];
	if (gptq && q->H && q->nsamp) {
		double *H = q->H, mean = 0;
		hd = malloc((size_t)K * sizeof *hd);
		for (int j = 0; j < K; j++) mean += H[j * K + j];
		mean /= K;
		for (int j = 0; j < K; j++) {
			if (H[j * K + j] == 0) {
				H[j * K + j] = 1;
				for (int c = 0; c < C; c++) W[(long)c * K + j] = 0;
			}
			H[j * K + j] += 0.01 * mean;
			hd[j] = H[j * K + j];
		}
		U = malloc((size_t)K * (size_t)K * sizeof *U);
		if (!inv_chol_upper(H, K, U)) {
			free(U);
			U = NULL;
		}
	}
	for (int c = 0; c < C; c++) {
		double *w = W + (long)c * K;
		double s = best_scale(w, K, hd, lim);
		x->qs[c] = (float)s;
		for (int j = 0; j < K; j++) {
			int code = code_of(w[j], s, lim);
			set_code(x, q, c, j, code);
			if (U) {
				double err = (w[j] - s * code) / U[j * K + j];
				for (int jj = j + 1; jj < K; jj++) w[jj] -= err * U[j * K + jj];
			}
		}
	}
	for (int c = 0; c < C; c++)
		for (int j = 0; j < K; j++) {
			long i = q->axis == 0 ? (long)c * K + j : (long)j * C + c;
			x->data[i] = (float)((double)tgo_qget(x->q, bits, i) * x->qs[c]);
		}
	if (log) {
		size_t l = strlen(log);
		snprintf(log + l, (size_t)logn - l, "%s int%d axis %d %s\n", x->name, bits, q->axis, U ? "gptq" : "rtn");
	}
	free(W);
	free(hd);
	free(U);
}

/* calib: ncalib rows of m->per floats (already parsed the way the reference
 * parses text rows, with strtof). Returns the number of quantized params, or
 * -1 when none is eligible. */
int tgo_quantize(tgo_module *m, int bits, int gptq, const float *calib, long ncalib, int min_size, char *log, int logn)
{
	if (log && logn > 0) log[0] = 0;
	QSet s = eligible(m, min_size);
	if (!s.n) return -1;
	if (gptq && calib && ncalib > 0) {
		for (int i = 0; i < s.n; i++)
			if (s.p[i].K <= 2048) s.p[i].H = calloc((size_t)s.p[i].K * (size_t)s.p[i].K, sizeof(double));
		float *arena = malloc((size_t)m->arena * sizeof *arena), *out = malloc((size_t)m->nout * sizeof *out);
		int *steps = malloc((size_t)(m->nthink ? m->nthink : 1) * sizeof *steps);
		tgo_matmul_hook = hook;
		tgo_hook_ctx = &s;
		for (long r = 0; r < ncalib; r++) tgo_run_row(m, calib + r * m->per, out, steps, arena);
		tgo_matmul_hook = NULL;
		tgo_hook_ctx = NULL;
		free(arena);
		free(out);
		free(steps);
	}
	for (int i = 0; i < s.n; i++) quantize_param(m, &s.p[i], bits, gptq, log, logn);
	int n = s.n;
	for (int i = 0; i < s.n; i++) free(s.p[i].H);
	free(s.p);
	m->fixed_ready = 0;
	return n;
}
