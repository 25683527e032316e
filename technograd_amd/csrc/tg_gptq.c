/* Model-level quantization of the backend (`tgc quantize`, src/quant.c).
 *
 * What has to match the reference byte for byte is observable: which params
 * are quantized, each channel's f32 scale and int codes, the dequantized data
 * and the report line. Codes are roundings of doubles, so every double that
 * feeds one must come out of the same operations in the same order as in
 * the reference (this file is compiled with -ffp-contract=off). The rules,
 * restated:
 *
 *   which params  rank 2, not quantized yet, at least min_size elements,
 *                 not named __*, not the model output, and every use of it
 *                 one operand of a matmul, always the same side: the left
 *                 operand gives one scale per row (axis 0), the right one
 *                 per column (axis 1); a think loop's init or yield, or a
 *                 scan's carries, slices or stacks naming it rule it out
 *                 (src/quant.c:42-89).
 *   the step      per channel: amax = max |w|; candidates amax (1 - 0.05 g) /
 *                 lim for g = 0..9, each scored by the sum over the channel in
 *                 input order of (w - step code)^2, times the damped Hessian
 *                 diagonal under GPTQ; the first smallest score wins; an
 *                 all-zero channel gets 1e-8 (:176-200).
 *   a code        nearbyint(w / step) clamped to +-lim (127 or 7).
 *   GPTQ          the Hessian's diagonal mean (summed in input order) times
 *                 0.01 added to the diagonal, inputs never active (a zero on
 *                 the diagonal) set to 1 first with their weights zeroed;
 *                 U the upper triangular factor with H^-1 = U^T U, reached
 *                 through H = L L^T, L^-1 by forward substitution, H^-1 =
 *                 L^-T L^-1 and a second factorisation; then, per channel in
 *                 input order, each code's rounding error divided by U[j][j]
 *                 and taken off every later input j' in proportion to
 *                 U[j][j'] (:203-316).
 *
 * Each factor entry is one running subtraction (or sum) over k in increasing
 * order, the order the reference evaluates it in; how the entries are swept
 * is this file's own: a team of threads shares each column's entries (a
 * barrier between columns), and the inverse is kept transposed so that every
 * running sum walks two contiguous rows. Channels are independent given U.
 *
 * The Hessians come from the device (tg_hip.cpp): the calibration pass
 * captures each eligible weight's other matmul operand in the order the
 * reference's hook sees it, and H[r][c] sums x_r x_c over the samples in that
 * order, so H is the reference's to the bit. The reference gives a Hessian
 * only to params of K <= 2048 inputs (src/quant.c:346); tg_hip_quantize_model
 * keeps that limit as its default (max_k = 2048), and max_k <= 0 lifts it. */
#include "tg_gptq.h"

#include <math.h>
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------- which params --- */

enum { AS_LEFT = 1, AS_RIGHT = 2, AS_OTHER = 4 };

static void mark(unsigned char *use, int nval, int v, int how)
{
	if (v >= 0 && v < nval) use[v] |= (unsigned char)how;
}

/* every value's uses in block b (nested bodies included), or-ed into use[] */
static void note_uses(const tgm_module *m, const tgm_block *b, unsigned char *use)
{
	for (int i = 0; i < b->len; i++) {
		const tgm_ins *in = &b->v[i];
		if (in->op == TGM_THINK) {
			mark(use, m->nval, in->init, AS_OTHER);
			mark(use, m->nval, in->yield, AS_OTHER);
			note_uses(m, in->body, use);
			continue;
		}
		if (in->op == TGM_SCAN) {
			for (int k = 0; k < in->nc; k++) mark(use, m->nval, in->cinit[k], AS_OTHER), mark(use, m->nval, in->cnext[k], AS_OTHER);
			for (int k = 0; k < in->nx; k++) mark(use, m->nval, in->x[k], AS_OTHER);
			for (int k = 0; k < in->ny; k++) mark(use, m->nval, in->y[k], AS_OTHER);
			note_uses(m, in->body, use);
			continue;
		}
		const int mm = in->op == TGM_MATMUL && in->na == 2 && in->a[0] != in->a[1];
		for (int j = 0; j < in->na; j++) {
			const int v = in->a[j];
			if (v < 0 || v >= m->nval) continue;
			mark(use, m->nval, v, mm && m->val[v].sh.rank == 2 ? (j == 0 ? AS_LEFT : AS_RIGHT) : AS_OTHER);
		}
	}
}

int tgq_eligible(const tgm_module *m, int min_size, tgq_param **out)
{
	unsigned char *use = calloc((size_t)(m->nval ? m->nval : 1), 1);
	tgq_param *list = NULL;
	int n = 0;
	if (!use) return -1;
	note_uses(m, &m->top, use);
	for (int v = 0; v < m->nval; v++) {
		const tgm_value *x = &m->val[v];
		if (x->kind != TGM_PARAM || x->qbits || x->sh.rank != 2 || x->n < min_size || m->output == v) continue;
		if (x->name && x->name[0] == '_' && x->name[1] == '_') continue;
		if (use[v] != AS_LEFT && use[v] != AS_RIGHT) continue; /* unused, both sides, or used otherwise */
		tgq_param *grown = realloc(list, (size_t)(n + 1) * sizeof *grown);
		if (!grown) {
			free(list);
			free(use);
			return -1;
		}
		list = grown;
		const int axis = use[v] == AS_LEFT ? 0 : 1;
		list[n] = (tgq_param){ .v = v, .axis = axis, .C = x->sh.dim[axis], .K = x->sh.dim[1 - axis] };
		n++;
	}
	free(use);
	*out = list;
	return n;
}

/* ------------------------------------------------------ thread team --- */

typedef struct Team Team;
typedef void (*team_fn)(Team *t, int id);
struct Team {
	int size;
	team_fn fn;
	void *ctx;
	pthread_barrier_t bar;
	pthread_mutex_t mu;
	pthread_cond_t cv;
	int state; /* 0: members wait; 1: run fn; -1: leave without running it */
};

typedef struct {
	Team *t;
	int id;
} Member;

static void *member_main(void *p)
{
	Member *w = p;
	Team *t = w->t;
	pthread_mutex_lock(&t->mu);
	while (t->state == 0) pthread_cond_wait(&t->cv, &t->mu);
	const int go = t->state > 0;
	pthread_mutex_unlock(&t->mu);
	if (go) t->fn(t, w->id);
	return NULL;
}

static void team_release(Team *t, int state)
{
	pthread_mutex_lock(&t->mu);
	t->state = state;
	pthread_cond_broadcast(&t->cv);
	pthread_mutex_unlock(&t->mu);
}

/* fn(t, id) on `size` threads, the caller being id 0; they may wait for each
 * other with team_sync. Members are held at a gate until all of them have
 * started; if one cannot start, the others leave and fn runs on the caller
 * alone (size 1). */
static void team_run(int size, team_fn fn, void *ctx)
{
	enum { MAXT = 64 };
	Team t;
	memset(&t, 0, sizeof t);
	t.size = size < 1 ? 1 : size > MAXT ? MAXT : size;
	t.fn = fn, t.ctx = ctx;
	if (t.size > 1 && pthread_mutex_init(&t.mu, NULL) == 0) {
		if (pthread_cond_init(&t.cv, NULL) == 0) {
			pthread_t th[MAXT];
			Member mem[MAXT];
			int started = 1;
			for (; started < t.size; started++) {
				mem[started] = (Member){ &t, started };
				if (pthread_create(&th[started], NULL, member_main, &mem[started])) break;
			}
			const int all = started == t.size && pthread_barrier_init(&t.bar, NULL, (unsigned)t.size) == 0;
			team_release(&t, all ? 1 : -1);
			if (all) fn(&t, 0);
			for (int i = 1; i < started; i++) pthread_join(th[i], NULL);
			if (all) pthread_barrier_destroy(&t.bar);
			pthread_cond_destroy(&t.cv);
			pthread_mutex_destroy(&t.mu);
			if (all) return;
		} else {
			pthread_mutex_destroy(&t.mu);
		}
	}
	t.size = 1;
	fn(&t, 0);
}

static void team_sync(Team *t)
{
	if (t->size > 1) pthread_barrier_wait(&t->bar);
}

/* ------------------------------------------------- dense row algebra --- */

/* acc - a[0] b[0] - a[1] b[1] - ... in that order */
static double less_dots(double acc, const double *a, const double *b, int n)
{
	for (int k = 0; k < n; k++) acc -= a[k] * b[k];
	return acc;
}

/* 0 + a[0] b[0] + a[1] b[1] + ... in that order */
static double dots(const double *a, const double *b, int n)
{
	double acc = 0;
	for (int k = 0; k < n; k++) acc += a[k] * b[k];
	return acc;
}

typedef struct {
	double *A; /* n x n, row-major; the lower triangle is read, L is left there */
	int n, ok;
} Factor;

/* H = L L^T, column by column: column j's diagonal from row j's entries left
 * of it, then its entries below (row i's entries left of column j against
 * row j's), those rows shared out over the team; the upper triangle cleared */
static void factor_member(Team *t, int id)
{
	Factor *f = t->ctx;
	const int n = f->n;
	double *A = f->A;
	for (int j = 0; j < n; j++) {
		double *rj = A + (size_t)j * n;
		const double piv = less_dots(rj[j], rj, rj, j); /* every member computes the same value */
		if (piv <= 0) {
			if (id == 0) f->ok = 0;
			return; /* every member sees the same pivot and leaves at the same column */
		}
		const double d = sqrt(piv);
		for (int i = j + 1 + id; i < n; i += t->size) {
			double *ri = A + (size_t)i * n;
			ri[j] = less_dots(ri[j], ri, rj, j) / d;
		}
		team_sync(t);
		if (id == 0) {
			rj[j] = d;
			for (int k = j + 1; k < n; k++) rj[k] = 0;
		}
		team_sync(t);
	}
}

static int lower_factor(double *A, int n, int threads)
{
	Factor f = { A, n, 1 };
	team_run(n >= 256 ? threads : 1, factor_member, &f);
	return f.ok;
}

typedef struct {
	const double *L;
	double *LiT; /* (L^-1)^T: row c holds column c of L^-1 */
	double *G;   /* lower triangle of L^-T L^-1 */
	int n;
} Inverse;

/* column c of L^-1 by forward substitution, into row c of LiT */
static void inverse_member(Team *t, int id)
{
	Inverse *v = t->ctx;
	const int n = v->n;
	for (int c = id; c < n; c += t->size) {
		double *out = v->LiT + (size_t)c * n;
		for (int i = c; i < n; i++) {
			const double *li = v->L + (size_t)i * n;
			out[i] = less_dots(i == c ? 1.0 : 0.0, li + c, out + c, i - c) / li[i];
		}
	}
}

/* G[j][i] = sum over k >= j of L^-1[k][i] L^-1[k][j] (j >= i), in k order */
static void gram_member(Team *t, int id)
{
	Inverse *v = t->ctx;
	const int n = v->n;
	for (int i = id; i < n; i += t->size) {
		const double *ci = v->LiT + (size_t)i * n;
		for (int j = i; j < n; j++) v->G[(size_t)j * n + i] = dots(ci + j, v->LiT + (size_t)j * n + j, n - j);
	}
}

/* U, upper, with H^-1 = U^T U: H = L L^T, G = L^-T L^-1 = H^-1, G = L2 L2^T, U = L2^T */
static int inverse_factor(const double *H, int n, double *U, int threads)
{
	double *L = malloc((size_t)n * n * sizeof *L), *LiT = calloc((size_t)n * n, sizeof *LiT);
	int ok = L && LiT;
	if (ok) {
		memcpy(L, H, (size_t)n * n * sizeof *L);
		ok = lower_factor(L, n, threads);
	}
	if (ok) {
		Inverse v = { L, LiT, U, n };
		team_run(threads, inverse_member, &v);
		team_run(threads, gram_member, &v);
		ok = lower_factor(U, n, threads);
	}
	if (ok)
		for (int i = 0; i < n; i++)
			for (int j = i + 1; j < n; j++) U[(size_t)i * n + j] = U[(size_t)j * n + i], U[(size_t)j * n + i] = 0;
	free(L);
	free(LiT);
	return ok;
}

/* ----------------------------------------------------------- channels --- */

static int rtn_code(double w, double step, int lim)
{
	if (step <= 0) return 0;
	const double r = nearbyint(w / step);
	return r > lim ? lim : r < -lim ? -lim : (int)r;
}

/* the channel's clip step: ten candidates, the first of the smallest weighted error */
static double clip_step(const double *w, int K, const double *hdiag, int lim)
{
	double amax = 0;
	for (int j = 0; j < K; j++) amax = fabs(w[j]) > amax ? fabs(w[j]) : amax;
	if (amax == 0) return 1e-8;
	double pick = amax / lim, low = INFINITY;
	for (int g = 0; g < 10; g++) {
		const double step = amax * (1.0 - 0.05 * g) / lim;
		double err = 0;
		for (int j = 0; j < K; j++) {
			const double r = w[j] - step * rtn_code(w[j], step, lim);
			err += r * r * (hdiag ? hdiag[j] : 1.0);
		}
		if (err < low) low = err, pick = step;
	}
	return pick;
}

typedef struct {
	double *W;            /* [C][K] working weights (GPTQ updates them) */
	const double *hdiag;  /* damped Hessian diagonal, or NULL */
	const double *U;      /* upper factor of H^-1, or NULL (RTN) */
	int C, K, lim;
	int *codes;           /* [C][K] */
	double *step;         /* [C] */
} Channels;

static void channel_member(Team *t, int id)
{
	Channels *q = t->ctx;
	const int K = q->K;
	for (int c = id; c < q->C; c += t->size) {
		double *w = q->W + (size_t)c * K;
		int *code = q->codes + (size_t)c * K;
		const double step = q->step[c] = clip_step(w, K, q->hdiag, q->lim);
		for (int j = 0; j < K; j++) {
			code[j] = rtn_code(w[j], step, q->lim);
			if (!q->U) continue;
			const double *uj = q->U + (size_t)j * K;
			const double e = (w[j] - step * code[j]) / uj[j];
			for (int l = j + 1; l < K; l++) w[l] -= e * uj[l];
		}
	}
}

/* the damped Hessian diagonal; inputs never active set to 1 with their weights zeroed */
static void damp(double *H, double *W, int C, int K, double *hdiag)
{
	double mean = 0;
	for (int j = 0; j < K; j++) mean += H[(size_t)j * K + j];
	mean /= K;
	for (int j = 0; j < K; j++) {
		double *hjj = &H[(size_t)j * K + j];
		if (*hjj == 0) {
			*hjj = 1;
			for (int c = 0; c < C; c++) W[(size_t)c * K + j] = 0;
		}
		*hjj += 0.01 * mean;
		hdiag[j] = *hjj;
	}
}

static void logf_append(char *log, size_t logn, const char *fmt, ...) __attribute__((format(printf, 3, 4)));
static void logf_append(char *log, size_t logn, const char *fmt, ...)
{
	const size_t at = strlen(log);
	va_list ap;
	va_start(ap, fmt);
	if (at < logn) vsnprintf(log + at, logn - at, fmt, ap);
	va_end(ap);
}

int tgq_quantize_param(tgm_module *m, tgq_param *q, int bits, int gptq, int threads, char *log, size_t logn)
{
	tgm_value *x = &m->val[q->v];
	const int lim = bits == 8 ? 127 : 7, C = q->C, K = q->K;
	const size_t n = (size_t)C * K, nbytes = bits == 8 ? n : (n + 1) / 2;
	/* element (channel c, input j) of the param's own layout */
	#define AT(c, j) (q->axis == 0 ? (size_t)(c) * K + (size_t)(j) : (size_t)(j) * C + (size_t)(c))
	double *W = malloc(n * sizeof *W), *step = malloc((size_t)C * sizeof *step), *hdiag = NULL, *U = NULL;
	int *codes = malloc(n * sizeof *codes);
	unsigned char *packed = calloc(nbytes, 1);
	float *scale = malloc((size_t)C * sizeof *scale);
	int rc = -1;
	if (!W || !step || !codes || !packed || !scale) goto done;
	for (int c = 0; c < C; c++)
		for (int j = 0; j < K; j++) W[(size_t)c * K + j] = x->data[AT(c, j)];
	if (gptq && q->H && q->nsamp) {
		hdiag = malloc((size_t)K * sizeof *hdiag);
		U = malloc((size_t)K * K * sizeof *U);
		if (!hdiag || !U) goto done;
		damp(q->H, W, C, K, hdiag);
		if (!inverse_factor(q->H, K, U, threads)) {
			logf_append(log, logn, "quantize: %s: Hessian not positive definite, using rtn\n", x->name);
			free(U);
			U = NULL;
		}
	}
	Channels ch = { W, hdiag, U, C, K, lim, codes, step };
	team_run(C >= 64 ? threads : 1, channel_member, &ch);
	/* codes into the param's layout (int4: low nibble first), scales to f32 */
	for (int c = 0; c < C; c++) {
		scale[c] = (float)step[c];
		for (int j = 0; j < K; j++) {
			const size_t i = AT(c, j);
			const unsigned v = (unsigned)codes[(size_t)c * K + j];
			if (bits == 8) packed[i] = (unsigned char)v;
			else packed[i >> 1] = (unsigned char)(i & 1 ? (packed[i >> 1] & 0x0fu) | (v << 4) : (packed[i >> 1] & 0xf0u) | (v & 0x0fu));
		}
	}
	/* the report's error against the original weights, then data = the dequantized values */
	double err2 = 0, norm2 = 0;
	for (int c = 0; c < C; c++)
		for (int j = 0; j < K; j++) {
			const size_t i = AT(c, j);
			const double orig = x->data[i], deq = (double)codes[(size_t)c * K + j] * scale[c];
			err2 += (orig - deq) * (orig - deq);
			norm2 += orig * orig;
			x->data[i] = (float)deq;
		}
	#undef AT
	x->qbits = bits;
	x->qaxis = q->axis;
	x->q = packed;
	x->qs = scale;
	packed = NULL;
	scale = NULL;
	logf_append(log, logn, "  %-12s (f32 %d %d) -> int%d, %d %s scales, %s, relative weight error %.4f\n", x->name, x->sh.dim[0],
		    x->sh.dim[1], bits, C, q->axis == 0 ? "row" : "column", U ? "gptq" : "rtn", norm2 > 0 ? sqrt(err2 / norm2) : 0.0);
	rc = 0;
done:
	free(W);
	free(step);
	free(hdiag);
	free(U);
	free(codes);
	free(packed);
	free(scale);
	return rc;
}
