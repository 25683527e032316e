/* TEST INFRASTRUCTURE ONLY — oracle f32 interpreter.
 *
 * Restates the reference interpreter's dispatch (src/vm.c:211-415) and the
 * f32 kernels it calls (runtime/tg_rt.h). Every output is computed with the
 * same operation order as the reference: products summed in order p = 0..k-1
 * starting from 0.0f (tg_rt.h:78-90, :132-151), no FMA contraction (this file
 * is compiled with -ffp-contract=off and no -march, as the reference's
 * `cc -std=c11 -O3` build), libm for transcendentals.
 *
 * Function map (reference -> here):
 *   tg_add..tg_min (tg_rt.h:26-37) + bin_simple/row broadcast (vm.c:225-242,
 *     ops.c:75-80) + tg_bin_bc/bcast_desc (tg_rt.h:398-417, util.c:172-214) -> bin()
 *   unary kernels (tg_rt.h:40-75)                   -> unary()
 *   tg_matmul (tg_rt.h:81-116), tg_bmm (:439-442)   -> matmul_f32()
 *   tg_qget (tg_rt.h:124-129)                       -> tgo_qget() (tgir.c)
 *   tg_matmul_qa / tg_matmul_qb (tg_rt.h:132-151)   -> matmul_qa() / matmul_qb()
 *   tg_softmax / tg_rmsnorm (tg_rt.h:154-175)       -> softmax() / rmsnorm()
 *   tg_sum / tg_mean (tg_rt.h:178-181), tg_transpose (:183-187), tg_outer
 *     (:190-194), tg_take (:316-323), tg_delta (:361-366)
 *   think (vm.c:383-411), scan (vm.c:364-382), q_axis_for (ops.c:310-320),
 *   matmul_dims (ops.c:62-73)
 *
 * Pinned by: tests/golden (outputs of the reference VM built from its
 * own sources by oracle/Makefile: byte-identical), the reference's known
 * answers (tests/cases/ops.expected, README.md:49-51 latent_reasoner,
 * tests/run.sh:374 halt steps), and brute-force checks in tests/. libm
 * results are pinned only because both builds call the same glibc. */
#include "tgo.h"

#include <math.h>
#include <string.h>

/* This file is compiled twice: as the f32 oracle (the reference's arithmetic),
 * and by vm64.c with TGO_F64 as the same interpreter in double precision,
 * which tests use as a high-precision truth (the same operations in the same
 * order on the same f32 params, constants and inputs, rounded to double). */
#ifdef TGO_F64
typedef double real;
#define LM(fn) fn
#define TGO_RUN_ROW tgo_run_row64
#else
typedef float real;
#define LM(fn) fn##f
#define TGO_RUN_ROW tgo_run_row
#endif

#ifndef TGO_F64
void (*tgo_matmul_hook)(void *ctx, const tgo_module *m, const tgo_ins *in, const float *a, const float *b);
void *tgo_hook_ctx;
#define ACC(v) (v)
#else
/* Test-only: 1 leaves the quantized matmuls' running sums in f32 (a planted
 * mistake that the f64 truth's own tests must catch). */
int tgo_plant64;
#define ACC(v) (tgo_plant64 == 1 ? (real)(float)(v) : (v))
#endif

typedef struct {
	const tgo_module *m;
	real *arena;
	const real *in;
	int *steps;
} VM;

static real *ptr(VM *vm, int v)
{
	const tgo_value *x = &vm->m->val[v];
	switch (x->kind) {
	case TGO_PARAM:
#ifdef TGO_F64
	case TGO_STATE: return x->d64;
#else
	case TGO_STATE: return x->data;
#endif
	case TGO_INPUT: {
		long off = 0;
		for (int i = 0; i < x->index; i++) off += vm->m->val[vm->m->inputs[i]].n;
		return (real *)vm->in + off;
	}
	}
	return vm->arena + x->off;
}

#ifndef TGO_F64
void tgo_matmul_dims(const tgo_shape *a, const tgo_shape *b, int *m, int *k, int *n, int *g)
{
	*g = a->rank == 3 && b->rank == 3 ? a->dim[0] : 1;
	*m = a->rank == 3 ? (*g > 1 || b->rank == 3 ? a->dim[1] : a->dim[0] * a->dim[1]) : a->rank == 2 ? a->dim[0] : 1;
	*k = a->dim[a->rank - 1];
	*n = b->rank >= 2 ? b->dim[b->rank - 1] : 1;
}

int tgo_q_axis_for(const tgo_module *m, int param, const tgo_ins *in)
{
	if (m->val[param].sh.rank != 2) return -1;
	if (in->op == O_MATMUL) {
		if (in->a[0] == param && in->a[1] != param) return 0;
		if (in->a[1] == param && in->a[0] != param) return 1;
	}
	return -1;
}

#endif

/* ---- binary elementwise ---- */

static real bop(int op, real x, real y)
{
	switch (op) {
	case O_ADD: return x + y;
	case O_SUB: return x - y;
	case O_MUL: return x * y;
	case O_DIV: return x / y;
	case O_MAX: return x > y ? x : y;
	default: return x < y ? x : y;
	}
}

static void kbin(int op, real *o, const real *a, int sa, const real *b, int sb, int n)
{
	for (int i = 0; i < n; i++) o[i] = bop(op, a[i * sa], b[i * sb]);
}

static int suffix(const tgo_shape *small, const tgo_shape *big)
{
	if (small->rank < 1 || small->rank >= big->rank) return 0;
	for (int i = 1; i <= small->rank; i++)
		if (small->dim[small->rank - i] != big->dim[big->rank - i]) return 0;
	return 1;
}

static int seq(const tgo_shape *a, const tgo_shape *b)
{
	if (a->rank != b->rank) return 0;
	for (int i = 0; i < a->rank; i++)
		if (a->dim[i] != b->dim[i]) return 0;
	return 1;
}

#ifndef TGO_F64
int tgo_bcast_desc(const tgo_shape *out, const tgo_shape *a, const tgo_shape *b, int *d)
{
	int r = out->rank, dim[TGO_MAXRANK], st[2][TGO_MAXRANK];
	const tgo_shape *ops[2] = { a, b };
	for (int k = 0; k < 2; k++) {
		long acc = 1;
		for (int i = r - 1; i >= 0; i--) {
			const tgo_shape *s = ops[k];
			int j = s ? i - (r - s->rank) : -1, n = j >= 0 ? s->dim[j] : 1;
			st[k][i] = n == 1 ? 0 : (int)acc;
			acc *= n;
		}
	}
	int nr = 0;
	for (int i = 0; i < r; i++) {
		if (out->dim[i] == 1) continue;
		if (nr > 0) {
			int p = nr - 1, ok = 1;
			for (int k = 0; k < 2; k++) {
				long merged = (long)st[k][i] * out->dim[i];
				if (!((st[k][p] == 0 && st[k][i] == 0) || (st[k][i] != 0 && st[k][p] == merged))) ok = 0;
			}
			if (ok) {
				dim[p] *= out->dim[i];
				st[0][p] = st[0][i];
				st[1][p] = st[1][i];
				continue;
			}
		}
		dim[nr] = out->dim[i];
		st[0][nr] = st[0][i];
		st[1][nr] = st[1][i];
		nr++;
	}
	if (nr == 0) {
		dim[0] = 1;
		st[0][0] = st[1][0] = 0;
		nr = 1;
	}
	d[0] = nr;
	for (int i = 0; i < nr; i++) {
		d[1 + i] = dim[i];
		d[1 + nr + i] = st[0][i];
		d[1 + 2 * nr + i] = st[1][i];
	}
	return 1 + 3 * nr;
}
#endif

static void bin(VM *vm, const tgo_ins *in, real *o, const real *a, const real *b)
{
	const tgo_module *m = vm->m;
	const tgo_shape *so = &m->val[in->out].sh, *s0 = &m->val[in->a[0]].sh, *s1 = &m->val[in->a[1]].sh;
	int n = tgo_numel(so), na = tgo_numel(s0), nb = tgo_numel(s1);
	int simple = ((na == n || na == 1) && (nb == n || nb == 1)) || (seq(s0, so) && suffix(s1, so)) || (seq(s1, so) && suffix(s0, so));
	if (!simple) {
		int d[1 + 3 * TGO_MAXRANK], idx[TGO_MAXRANK] = { 0 };
		tgo_bcast_desc(so, s0, s1, d);
		int r = d[0];
		const int *dim = d + 1, *sa = d + 1 + r, *sb = d + 1 + 2 * r;
		int w = dim[r - 1];
		long cnt = 1, ia = 0, ib = 0;
		for (int i = 0; i < r - 1; i++) cnt *= dim[i];
		for (long i = 0; i < cnt; i++) {
			kbin(in->op, o + i * w, a + ia, sa[r - 1] != 0, b + ib, sb[r - 1] != 0, w);
			for (int x = r - 2; x >= 0; x--) {
				ia += sa[x];
				ib += sb[x];
				if (++idx[x] < dim[x]) break;
				ia -= (long)sa[x] * dim[x];
				ib -= (long)sb[x] * dim[x];
				idx[x] = 0;
			}
		}
	} else if ((na == n || na == 1) && (nb == n || nb == 1)) {
		kbin(in->op, o, a, na == n, b, nb == n, n);
	} else {
		int w = na < n ? na : nb;
		for (int r = 0; r < n / w; r++) kbin(in->op, o + r * w, na < n ? a : a + r * w, 1, nb < n ? b : b + r * w, 1, w);
	}
}

/* ---- unary elementwise ---- */

static void unary(int op, real *o, const real *a, int n)
{
	for (int i = 0; i < n; i++) {
		real x = a[i];
		switch (op) {
		case O_NEG: o[i] = -x; break;
		case O_TANH: o[i] = LM(tanh)(x); break;
		case O_RELU: o[i] = x > 0.0f ? x : 0.0f; break;
		case O_SIGMOID: o[i] = 1.0f / (1.0f + LM(exp)(-x)); break;
		case O_EXP: o[i] = LM(exp)(x); break;
		case O_SQRT: o[i] = LM(sqrt)(x); break;
		case O_GELU: o[i] = 0.5f * x * (1.0f + LM(tanh)(0.7978845608f * (x + 0.044715f * x * x * x))); break;
		case O_SILU: o[i] = x / (1.0f + LM(exp)(-x)); break;
		case O_SOFTPLUS: o[i] = (x > 0.0f ? x : 0.0f) + LM(log1p)(LM(exp)(-LM(fabs)(x))); break;
		case O_LOG: o[i] = LM(log)(x); break;
		case O_SIN: o[i] = LM(sin)(x); break;
		case O_COS: o[i] = LM(cos)(x); break;
		case O_FLOOR: o[i] = LM(floor)(x); break;
		case O_STEP: o[i] = x > 0.0f ? 1.0f : 0.0f; break;
		}
	}
}

/* ---- matmuls ---- */

static void matmul_f32(real *o, const real *a, const real *b, int m, int k, int n)
{
	for (int i = 0; i < m; i++)
		for (int j = 0; j < n; j++) {
			real s = 0.0f;
			for (int p = 0; p < k; p++) s += a[(long)i * k + p] * b[(long)p * n + j];
			o[(long)i * n + j] = s;
		}
}

static void matmul_qa(real *o, const signed char *q, int bits, const float *s, const real *b, int m, int k, int n)
{
	for (int i = 0; i < m; i++)
		for (int j = 0; j < n; j++) {
			real acc = 0.0f;
			for (int p = 0; p < k; p++) acc = ACC(acc + (real)tgo_qget(q, bits, (long)i * k + p) * b[(long)p * n + j]);
			o[(long)i * n + j] = s[i] * acc;
		}
}

static void matmul_qb(real *o, const real *a, const signed char *q, int bits, const float *s, int m, int k, int n)
{
	for (int i = 0; i < m; i++)
		for (int j = 0; j < n; j++) {
			real acc = 0.0f;
			for (int p = 0; p < k; p++) acc = ACC(acc + a[(long)i * k + p] * (real)tgo_qget(q, bits, (long)p * n + j));
			o[(long)i * n + j] = s[j] * acc;
		}
}

/* ---- row ops ---- */

static void softmax(real *o, const real *a, int rows, int cols)
{
	for (int r = 0; r < rows; r++) {
		const real *x = a + (long)r * cols;
		real *y = o + (long)r * cols;
		real mx = x[0], s = 0.0f;
		for (int i = 1; i < cols; i++)
			if (x[i] > mx) mx = x[i];
		for (int i = 0; i < cols; i++) {
			y[i] = LM(exp)(x[i] - mx);
			s += y[i];
		}
		for (int i = 0; i < cols; i++) y[i] /= s;
	}
}

static void rmsnorm(real *o, const real *a, int rows, int cols)
{
	for (int r = 0; r < rows; r++) {
		const real *x = a + (long)r * cols;
		real *y = o + (long)r * cols;
		real s = 0.0f;
		for (int i = 0; i < cols; i++) s += x[i] * x[i];
		real inv = 1.0f / LM(sqrt)(s / (real)cols + 1e-6f);
		for (int i = 0; i < cols; i++) y[i] = x[i] * inv;
	}
}

static real delta(const real *a, const real *b, int n)
{
	real d = 0.0f;
	for (int i = 0; i < n; i++) {
		real e = LM(fabs)(a[i] - b[i]);
		if (e > d) d = e;
	}
	return d;
}

static void copy(real *o, const real *a, long n)
{
	if (o != a) memmove(o, a, (size_t)n * sizeof *o);
}

static void exec(VM *vm, const tgo_block *b);

static void exec_one(VM *vm, const tgo_ins *in)
{
	const tgo_module *m = vm->m;
	if (in->op == O_SCAN) {
		for (int k = 0; k < in->nc; k++) copy(ptr(vm, in->c[k]), ptr(vm, in->cinit[k]), m->val[in->c[k]].n);
		for (int step = 0; step < in->T; step++) {
			int t = in->reverse ? in->T - 1 - step : step;
			for (int j = 0; j < in->nx; j++) {
				int w = m->val[in->xt[j]].n;
				copy(ptr(vm, in->xt[j]), ptr(vm, in->x[j]) + (long)t * w, w);
			}
			exec(vm, in->body);
			for (int y = 0; y < in->ny; y++) {
				int w = m->val[in->y[y]].n;
				copy(ptr(vm, in->ys[y]) + (long)t * w, ptr(vm, in->y[y]), w);
			}
			for (int k = 0; k < in->nc; k++) copy(ptr(vm, in->c[k]), ptr(vm, in->cnext[k]), m->val[in->c[k]].n);
		}
		if (in->stid >= 0) vm->steps[in->stid] = in->T;
		return;
	}
	real *o = ptr(vm, in->out);
	int n = m->val[in->out].n;
	const real *a = in->na > 0 ? ptr(vm, in->a[0]) : NULL;
	const real *c = in->na > 1 ? ptr(vm, in->a[1]) : NULL;
	switch (in->op) {
	case O_CONST: o[0] = in->k; break;
	case O_ADD: case O_SUB: case O_MUL: case O_DIV: case O_MAX: case O_MIN: bin(vm, in, o, a, c); break;
	case O_NEG: case O_TANH: case O_RELU: case O_SIGMOID: case O_EXP: case O_SQRT: case O_GELU: case O_SILU:
	case O_SOFTPLUS: case O_LOG: case O_SIN: case O_COS: case O_FLOOR: case O_STEP: unary(in->op, o, a, n); break;
	case O_MATMUL: {
		int mm, kk, nn, gg;
		const tgo_value *qa = &m->val[in->a[0]], *qb = &m->val[in->a[1]];
		tgo_matmul_dims(&qa->sh, &qb->sh, &mm, &kk, &nn, &gg);
		if (gg > 1) {
			for (int g = 0; g < gg; g++)
				matmul_f32(o + (long)g * mm * nn, a + (long)g * mm * kk, c + (long)g * kk * nn, mm, kk, nn);
			break;
		}
#ifndef TGO_F64
		if (tgo_matmul_hook) tgo_matmul_hook(tgo_hook_ctx, m, in, a, c);
#endif
		if (qa->qbits && tgo_q_axis_for(m, in->a[0], in) == qa->qaxis) matmul_qa(o, qa->q, qa->qbits, qa->qs, c, mm, kk, nn);
		else if (qb->qbits && tgo_q_axis_for(m, in->a[1], in) == qb->qaxis) matmul_qb(o, a, qb->q, qb->qbits, qb->qs, mm, kk, nn);
		else matmul_f32(o, a, c, mm, kk, nn);
		break;
	}
	case O_SOFTMAX:
	case O_RMSNORM: {
		const tgo_shape *s = &m->val[in->a[0]].sh;
		int cols = s->rank ? s->dim[s->rank - 1] : 1, rows = tgo_numel(s) / cols;
		if (in->op == O_SOFTMAX) softmax(o, a, rows, cols);
		else rmsnorm(o, a, rows, cols);
		break;
	}
	case O_SUM:
	case O_MEAN: {
		int k = m->val[in->a[0]].n;
		real s = 0.0f;
		for (int i = 0; i < k; i++) s += a[i];
		o[0] = in->op == O_SUM ? s : s / (real)k;
		break;
	}
	case O_TRANSPOSE: {
		const tgo_shape *s = &m->val[in->a[0]].sh;
		int g = s->rank == 3 ? s->dim[0] : 1, r = s->dim[s->rank - 2], cc = s->dim[s->rank - 1];
		for (int z = 0; z < g; z++)
			for (int i = 0; i < r; i++)
				for (int j = 0; j < cc; j++) o[(long)z * r * cc + (long)j * r + i] = a[(long)z * r * cc + (long)i * cc + j];
		break;
	}
	case O_OUTER: {
		int mm = m->val[in->a[0]].n, nn = m->val[in->a[1]].n;
		for (int i = 0; i < mm; i++)
			for (int j = 0; j < nn; j++) o[(long)i * nn + j] = a[i] * c[j];
		break;
	}
	case O_RESHAPE: copy(o, a, n); break;
	case O_TAKE: {
		const tgo_shape *s0 = &m->val[in->a[0]].sh;
		int cnt = m->val[in->a[1]].sh.dim[0], d = s0->dim[0], h = tgo_numel(s0) / s0->dim[0];
		for (int i = 0; i < cnt; i++) {
			real rr = LM(floor)(c[i] + 0.5f);
			int t = rr >= 0.0f && rr < (real)d ? (int)rr : -1;
			for (int j = 0; j < h; j++) o[(long)i * h + j] = t >= 0 ? a[(long)t * h + j] : 0.0f;
		}
		break;
	}
	case O_THINK: {
		copy(o, ptr(vm, in->init), n);
		int it = 0;
		real survive = 1.0f;
		while (it < in->maxit) {
			exec(vm, in->body);
			it++;
			const real *y = ptr(vm, in->yield);
			real d = delta(y, o, n);
			copy(o, y, n);
			if (in->eps >= 0 && d <= in->eps) break;
			if (in->halt >= 0) {
				real p = *ptr(vm, in->halt);
				survive *= 1.0f - (p < 0.0f ? 0.0f : p > 1.0f ? 1.0f : p);
				if (1.0f - survive > in->hthr) break;
			}
		}
		vm->steps[in->tid] = it;
		break;
	}
	}
}

static void exec(VM *vm, const tgo_block *b)
{
	for (int i = 0; i < b->len; i++) exec_one(vm, &b->v[i]);
}

void TGO_RUN_ROW(const tgo_module *m, const real *in, real *out, int *steps, real *arena)
{
	VM vm = { m, arena, in, steps };
	exec(&vm, &m->top);
	copy(out, ptr(&vm, m->output), m->nout);
}
