/* Model-level quantization of the backend (`tgc quantize`, src/quant.c):
 * which params are quantized, their scales and codes, RTN or GPTQ. The
 * calibration Hessians come from the device (tg_hip.cpp: the row program
 * captures each eligible weight's other matmul operand in the order the
 * reference's hook sees it, and one thread per element sums x_r x_c over the
 * samples in that order, so H is the reference's to the bit); everything
 * here is host double arithmetic in the reference's operation order
 * (compiled with -ffp-contract=off), parallel only over independent results:
 *   eligibility  rank-2 params with at least min_size elements, not named
 *                __*, not the output, used only as a matmul operand with one
 *                axis (left: per-row scales, axis 0; right: per column, 1)
 *                (src/quant.c:42-89);
 *   scale        per channel, the clip of absmax (ten candidates) that
 *                minimises the rounding error, weighted by the damped
 *                Hessian diagonal under GPTQ (:184-200);
 *   GPTQ         H + 0.01 mean(diag) on the diagonal, inputs never active
 *                zeroed, U = the upper Cholesky factor of H^-1 through two
 *                Cholesky factorisations and a triangular inverse (:203-253),
 *                then per channel, input by input, each rounding error pushed
 *                onto the remaining inputs (:258-316). Channels are
 *                independent given U, and so are the rows of each Cholesky
 *                step and the columns of the inverse: those run on threads.
 * The reference quantizes with GPTQ only for K <= 2048 (src/quant.c:346);
 * here every eligible param gets its Hessian, K included up to 8192. */
#include "tg_gptq.h"

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------- eligibility --- */

static int q_axis_for(const tgm_module *m, int v, const tgm_ins *in)
{
	if (m->val[v].sh.rank != 2) return -1;
	if (in->op == TGM_MATMUL) {
		if (in->a[0] == v && in->a[1] != v) return 0;
		if (in->a[1] == v && in->a[0] != v) return 1;
	}
	return -1;
}

static int use_axis(const tgm_module *m, int v, const tgm_block *b, int *axis)
{
	for (int i = 0; i < b->len; i++) {
		const tgm_ins *in = &b->v[i];
		if (in->op == TGM_THINK) {
			if (in->init == v || in->yield == v || !use_axis(m, v, in->body, axis)) return 0;
		} else if (in->op == TGM_SCAN) {
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
				int a = q_axis_for(m, v, in);
				if (a < 0 || (*axis >= 0 && *axis != a)) return 0;
				*axis = a;
			}
		}
	}
	return 1;
}

int tgq_eligible(const tgm_module *m, int min_size, tgq_param **out)
{
	int n = 0;
	tgq_param *p = NULL;
	for (int v = 0; v < m->nval; v++) {
		const tgm_value *x = &m->val[v];
		if (x->kind != TGM_PARAM || x->qbits || x->sh.rank != 2 || x->n < min_size) continue;
		if (x->name && !strncmp(x->name, "__", 2)) continue;
		if (m->output == v) continue;
		int axis = -1;
		if (!use_axis(m, v, &m->top, &axis) || axis < 0) continue;
		tgq_param *np = realloc(p, (size_t)(n + 1) * sizeof *np);
		if (!np) {
			free(p);
			return -1;
		}
		p = np;
		memset(&p[n], 0, sizeof *p);
		p[n].v = v;
		p[n].axis = axis;
		p[n].C = x->sh.dim[axis];
		p[n].K = x->sh.dim[1 - axis];
		n++;
	}
	*out = p;
	return n;
}

/* ------------------------------------------------------------- threads --- */

typedef struct {
	void (*fn)(void *ctx, int lo, int hi);
	void *ctx;
	int lo, hi;
} Part;

static void *part_main(void *a)
{
	Part *p = a;
	p->fn(p->ctx, p->lo, p->hi);
	return NULL;
}

/* fn over [0, n) in contiguous parts, one per thread */
static void par(int n, int threads, void (*fn)(void *, int, int), void *ctx)
{
	if (threads > 64) threads = 64;
	if (threads < 1 || n < 64) threads = 1;
	Part parts[64];
	pthread_t th[64];
	int ok[64] = { 0 };
	for (int t = 0; t < threads; t++) parts[t] = (Part){ fn, ctx, (int)((long)n * t / threads), (int)((long)n * (t + 1) / threads) };
	for (int t = 1; t < threads; t++) ok[t] = pthread_create(&th[t], NULL, part_main, &parts[t]) == 0;
	fn(ctx, parts[0].lo, parts[0].hi);
	for (int t = 1; t < threads; t++) {
		if (ok[t]) pthread_join(th[t], NULL);
		else fn(ctx, parts[t].lo, parts[t].hi);
	}
}

/* ---------------------------------------------------------- Cholesky --- */

typedef struct {
	double *A;
	const double *L;
	double *Li, *U;
	int n, j, c;
} Ch;

static void chol_rows(void *p, int lo, int hi) /* rows j+1+lo .. of column j */
{
	Ch *c = p;
	const int n = c->n, j = c->j;
	double *A = c->A, d = A[j * n + j];
	for (int i = j + 1 + lo; i < j + 1 + hi; i++) {
		double s = A[i * n + j];
		for (int k = 0; k < j; k++) s -= A[i * n + k] * A[j * n + k];
		A[i * n + j] = s / d;
	}
}

/* lower Cholesky factor in place (src/quant.c:203-220): column j's diagonal,
 * then its rows below (independent of each other), then zeros above */
static int cholesky(double *A, int n, int threads)
{
	Ch c = { A, NULL, NULL, NULL, n, 0, 0 };
	for (int j = 0; j < n; j++) {
		double d = A[j * n + j];
		for (int k = 0; k < j; k++) d -= A[j * n + k] * A[j * n + k];
		if (d <= 0) return 0;
		A[j * n + j] = sqrt(d);
		c.j = j;
		par(n - j - 1, (n - j - 1) >= 256 ? threads : 1, chol_rows, &c);
		for (int k = j + 1; k < n; k++) A[j * n + k] = 0;
	}
	return 1;
}

static void inv_cols(void *p, int lo, int hi) /* columns of L^-1 by forward substitution */
{
	Ch *c = p;
	const int n = c->n;
	const double *L = c->L;
	double *Li = c->Li;
	for (int col = lo; col < hi; col++)
		for (int i = col; i < n; i++) {
			double s = i == col ? 1.0 : 0.0;
			for (int k = col; k < i; k++) s -= L[i * n + k] * Li[k * n + col];
			Li[i * n + col] = s / L[i * n + i];
		}
}

static void hinv_rows(void *p, int lo, int hi) /* H^-1 = Li^T Li, upper triangle by rows, mirrored */
{
	Ch *c = p;
	const int n = c->n;
	const double *Li = c->Li;
	double *U = c->U;
	for (int i = lo; i < hi; i++)
		for (int j = i; j < n; j++) {
			double s = 0;
			for (int k = j; k < n; k++) s += Li[k * n + i] * Li[k * n + j];
			U[i * n + j] = U[j * n + i] = s;
		}
}

/* U, upper with H^-1 = U^T U (src/quant.c:222-253) */
static int inv_chol_upper(const double *H, int n, double *U, int threads)
{
	double *L = malloc((size_t)n * n * sizeof *L), *Li = calloc((size_t)n * n, sizeof *Li);
	int ok = L && Li;
	if (ok) {
		memcpy(L, H, (size_t)n * n * sizeof *L);
		ok = cholesky(L, n, threads);
	}
	if (ok) {
		Ch c = { NULL, L, Li, U, n, 0, 0 };
		par(n, threads, inv_cols, &c);
		par(n, threads, hinv_rows, &c);
		ok = cholesky(U, n, threads);
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

/* ------------------------------------------------------------ channels --- */

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

typedef struct {
	double *W;
	const double *hd, *U;
	int K, lim;
	int *codes; /* [C][K] */
	double *scale;
} Chan;

static void channels(void *p, int lo, int hi)
{
	Chan *c = p;
	const int K = c->K;
	for (int ch = lo; ch < hi; ch++) {
		double *w = c->W + (size_t)ch * K;
		double s = best_scale(w, K, c->hd, c->lim);
		c->scale[ch] = s;
		for (int j = 0; j < K; j++) {
			int code = code_of(w[j], s, c->lim);
			c->codes[(size_t)ch * K + j] = code;
			if (c->U) { /* this input's rounding error, pushed onto the remaining inputs */
				double err = (w[j] - s * code) / c->U[(size_t)j * K + j];
				for (int jj = j + 1; jj < K; jj++) w[jj] -= err * c->U[(size_t)j * K + jj];
			}
		}
	}
}

int tgq_quantize_param(tgm_module *m, tgq_param *q, int bits, int gptq, int threads, char *log, size_t logn)
{
	tgm_value *x = &m->val[q->v];
	const int lim = bits == 8 ? 127 : 7, C = q->C, K = q->K;
	const long n = (long)C * K;
	double *W = malloc((size_t)n * sizeof *W), *hd = NULL, *U = NULL, *scale = malloc((size_t)C * sizeof *scale);
	int *codes = malloc((size_t)n * sizeof *codes);
	unsigned char *qb = calloc((size_t)(bits == 8 ? n : (n + 1) / 2), 1);
	float *qs = malloc((size_t)C * sizeof *qs);
	int rc = -1;
	const char *how = "rtn";
	if (!W || !scale || !codes || !qb || !qs) goto out;
	for (int c = 0; c < C; c++)
		for (int j = 0; j < K; j++) W[(size_t)c * K + j] = q->axis == 0 ? x->data[(size_t)c * K + j] : x->data[(size_t)j * C + c];
	if (gptq && q->H && q->nsamp) {
		double *H = q->H, mean = 0;
		hd = malloc((size_t)K * sizeof *hd);
		U = malloc((size_t)K * K * sizeof *U);
		if (!hd || !U) goto out;
		for (int j = 0; j < K; j++) mean += H[(size_t)j * K + j];
		mean /= K;
		for (int j = 0; j < K; j++) {
			if (H[(size_t)j * K + j] == 0) { /* an input never active: its weights do not matter */
				H[(size_t)j * K + j] = 1;
				for (int c = 0; c < C; c++) W[(size_t)c * K + j] = 0;
			}
			H[(size_t)j * K + j] += 0.01 * mean; /* dampening */
			hd[j] = H[(size_t)j * K + j];
		}
		if (inv_chol_upper(H, K, U, threads)) {
			how = "gptq";
		} else {
			size_t o = strlen(log);
			snprintf(log + o, logn - o, "quantize: %s: Hessian not positive definite, using rtn\n", x->name);
			free(U);
			U = NULL;
		}
	}
	Chan ch = { W, hd, U, K, lim, codes, scale };
	par(C, threads, channels, &ch);
	double num = 0, den = 0;
	for (int c = 0; c < C; c++) {
		qs[c] = (float)scale[c];
		for (int j = 0; j < K; j++) {
			long i = q->axis == 0 ? (long)c * K + j : (long)j * C + c;
			int code = codes[(size_t)c * K + j];
			if (bits == 8) qb[i] = (unsigned char)(signed char)code;
			else if (i & 1) qb[i >> 1] = (unsigned char)((qb[i >> 1] & 0x0f) | ((unsigned)code << 4));
			else qb[i >> 1] = (unsigned char)((qb[i >> 1] & 0xf0) | (code & 0x0f));
		}
	}
	for (int c = 0; c < C; c++) /* report against the original weights; data becomes the dequantized values */
		for (int j = 0; j < K; j++) {
			long i = q->axis == 0 ? (long)c * K + j : (long)j * C + c;
			double w0 = x->data[i], wq = (double)codes[(size_t)c * K + j] * qs[c];
			num += (w0 - wq) * (w0 - wq);
			den += w0 * w0;
			x->data[i] = (float)wq;
		}
	x->qbits = bits;
	x->qaxis = q->axis;
	x->q = qb;
	x->qs = qs;
	qb = NULL;
	qs = NULL;
	{
		size_t o = strlen(log);
		snprintf(log + o, logn - o, "  %-12s (f32 %d %d) -> int%d, %d %s scales, %s, relative weight error %.4f\n", x->name, x->sh.dim[0],
			 x->sh.dim[1], bits, C, q->axis == 0 ? "row" : "column", how, den > 0 ? sqrt(num / den) : 0.0);
	}
	rc = 0;
out:
	free(W);
	free(hd);
	free(U);
	free(scale);
	free(codes);
	free(qb);
	free(qs);
	return rc;
}
