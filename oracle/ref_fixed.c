/* TEST INFRASTRUCTURE ONLY — Q16.16 execution with the reference's own kernels,
 * kept as a cross-check of the emitted units.
 *
 * The Q16.16 goldens come from the reference's `tgc c --fixed` unit itself
 * (src/cgen.c compiled into oracle/_ref; `tgc_ref c`). This file is a second,
 * independent route to the same numbers: it includes runtime/tg_rtq.h from
 * /root/reference unchanged and walks the reference's own Module (loaded and
 * planned by the reference's load_module and plan) issuing the kernel calls
 * the emitted unit makes, with the same conversions: params to_fixed(v, 16),
 * quant scales to_fixed(s, 24) as Q7.24, constants to_fixed(k, 16), think
 * thresholds kept positive (cgen.c:76-89, :286-290, :295-305, :435-455).
 * Arena offsets are the reference planner's. tests/golden/make_golden.py
 * requires both routes to agree bit for bit before it writes a fixture. */
#include "tg.h"
#include "tg_rtq.h"

#include <math.h>
#include <stdlib.h>

static tg_t **pfx;   /* Q16.16 param values by value index */
static int32_t **pqs; /* Q7.24 scales by value index */

static long long to_fixed(double v, int frac)
{
	double s = v * (double)(1LL << frac);
	if (s >= 2147483647.0) return 2147483647LL;
	if (s <= -2147483648.0) return -2147483647LL - 1;
	return llround(s);
}

void ref_fixed_prepare(const Module *m)
{
	pfx = calloc((size_t)m->nval, sizeof *pfx);
	pqs = calloc((size_t)m->nval, sizeof *pqs);
	for (int v = 0; v < m->nval; v++) {
		const Value *x = &m->val[v];
		if (x->kind != V_PARAM && x->kind != V_STATE) continue;
		int n = shape_numel(&x->sh);
		pfx[v] = malloc((size_t)n * sizeof(tg_t));
		for (int i = 0; i < n; i++) pfx[v][i] = (tg_t)to_fixed(x->data[i], 16);
		if (x->qbits) {
			int nch = x->sh.dim[x->qaxis];
			pqs[v] = malloc((size_t)nch * sizeof(int32_t));
			for (int i = 0; i < nch; i++) pqs[v][i] = (int32_t)to_fixed(x->qs[i], 24);
		}
	}
}

typedef struct {
	const Module *m;
	tg_t *A;
	const tg_t *in;
	int *steps;
} FX;

static tg_t *ptr(FX *f, int v)
{
	const Value *x = &f->m->val[v];
	if (x->kind == V_PARAM || x->kind == V_STATE) return pfx[v];
	if (x->kind == V_INPUT) {
		int off = 0;
		for (int i = 0; i < x->index; i++) off += shape_numel(&f->m->val[f->m->inputs[i]].sh);
		return (tg_t *)f->in + off;
	}
	return f->A + x->off;
}

static void block(FX *f, const Block *b)
{
	const Module *m = f->m;
	for (int i = 0; i < b->len; i++) {
		const Ins *in = &b->v[i];
		int n = shape_numel(&m->val[in->out].sh);
		tg_t *o = ptr(f, in->out);
		const tg_t *a = in->na > 0 ? ptr(f, in->a[0]) : NULL, *c = in->na > 1 ? ptr(f, in->a[1]) : NULL;
		switch (tg_ops[in->op].cls) {
		case CLS_CONST: o[0] = (tg_t)to_fixed(in->k, 16); break;
		case CLS_BIN: {
			void (*k)(tg_t *, const tg_t *, int, const tg_t *, int, int) = in->op == OP_ADD ? tg_add : in->op == OP_SUB ? tg_sub
				: in->op == OP_MUL ? tg_mul : in->op == OP_DIV ? tg_div : in->op == OP_MAX ? tg_max : tg_min;
			int na = shape_numel(&m->val[in->a[0]].sh), nb = shape_numel(&m->val[in->a[1]].sh);
			if (!bin_simple(&m->val[in->out].sh, &m->val[in->a[0]].sh, &m->val[in->a[1]].sh)) {
				int d[TG_BCAST_DESC];
				bcast_desc(&m->val[in->out].sh, &m->val[in->a[0]].sh, &m->val[in->a[1]].sh, d);
				tg_bin_bc(in->op - OP_ADD, o, a, c, d);
			} else if ((na == n || na == 1) && (nb == n || nb == 1)) {
				k(o, a, na == n, c, nb == n, n);
			} else {
				int w = na < n ? na : nb;
				for (int r = 0; r < n / w; r++) k(o + r * w, na < n ? a : a + r * w, 1, nb < n ? c : c + r * w, 1, w);
			}
			break;
		}
		case CLS_UN:
			switch (in->op) {
			case OP_NEG: tg_neg(o, a, n); break;
			case OP_TANH: tg_tanh(o, a, n); break;
			case OP_RELU: tg_relu(o, a, n); break;
			case OP_SIGMOID: tg_sigmoid(o, a, n); break;
			case OP_EXP: tg_exp(o, a, n); break;
			case OP_SQRT: tg_sqrt(o, a, n); break;
			case OP_GELU: tg_gelu(o, a, n); break;
			case OP_SILU: tg_silu(o, a, n); break;
			case OP_SOFTPLUS: tg_softplus(o, a, n); break;
			case OP_LOG: tg_log(o, a, n); break;
			case OP_STEP: tg_step(o, a, n); break;
			case OP_SIN: tg_sin(o, a, n); break;
			case OP_FLOOR: tg_floor(o, a, n); break;
			case OP_COS: tg_cos(o, a, n); break;
			default: abort();
			}
			break;
		case CLS_MATMUL: {
			int mm, kk, nn;
			matmul_dims(&m->val[in->a[0]].sh, &m->val[in->a[1]].sh, &mm, &kk, &nn);
			int gg = matmul_groups(&m->val[in->a[0]].sh, &m->val[in->a[1]].sh);
			const Value *qa = &m->val[in->a[0]], *qb = &m->val[in->a[1]];
			if (gg > 1) tg_bmm(o, a, c, gg, mm, kk, nn);
			else if (qa->qbits && q_axis_for(m, in->a[0], in) == qa->qaxis) tg_matmul_qa(o, qa->q, qa->qbits, pqs[in->a[0]], c, mm, kk, nn);
			else if (qb->qbits && q_axis_for(m, in->a[1], in) == qb->qaxis) tg_matmul_qb(o, a, qb->q, qb->qbits, pqs[in->a[1]], mm, kk, nn);
			else tg_matmul(o, a, c, mm, kk, nn);
			break;
		}
		case CLS_ROW: {
			int rows, cols;
			row_dims(&m->val[in->a[0]].sh, &rows, &cols);
			if (in->op == OP_SOFTMAX) tg_softmax(o, a, rows, cols);
			else tg_rmsnorm(o, a, rows, cols);
			break;
		}
		case CLS_RED:
			if (in->op == OP_SUM) tg_sum(o, a, shape_numel(&m->val[in->a[0]].sh));
			else tg_mean(o, a, shape_numel(&m->val[in->a[0]].sh));
			break;
		case CLS_OUTER: tg_outer(o, a, c, shape_numel(&m->val[in->a[0]].sh), shape_numel(&m->val[in->a[1]].sh)); break;
		case CLS_TRANS: {
			const Shape *s = &m->val[in->a[0]].sh;
			if (s->rank == 3) tg_btranspose(o, a, s->dim[0], s->dim[1], s->dim[2]);
			else tg_transpose(o, a, s->dim[0], s->dim[1]);
			break;
		}
		case CLS_RESHAPE: tg_copy(o, a, n); break;
		case CLS_ROWS: {
			const Shape *s0 = &m->val[in->a[0]].sh;
			if (in->op != OP_TAKE) abort();
			tg_take(o, a, c, m->val[in->a[1]].sh.dim[0], s0->dim[0], shape_numel(s0) / s0->dim[0]);
			break;
		}
		case CLS_SCAN: {
			const Scan *s = in->sc;
			for (int k = 0; k < s->nc; k++) tg_copy(ptr(f, s->c[k]), ptr(f, s->init[k]), shape_numel(&m->val[s->c[k]].sh));
			for (int st = 0; st < s->T; st++) {
				int t = s->reverse ? s->T - 1 - st : st;
				for (int j = 0; j < s->nx; j++) {
					int w = shape_numel(&m->val[s->xt[j]].sh);
					tg_copy(ptr(f, s->xt[j]), ptr(f, s->x[j]) + t * w, w);
				}
				block(f, in->body);
				for (int y = 0; y < s->ny; y++) {
					int w = shape_numel(&m->val[s->y[y]].sh);
					tg_copy(ptr(f, s->ys[y]) + t * w, ptr(f, s->y[y]), w);
				}
				for (int k = 0; k < s->nc; k++) tg_copy(ptr(f, s->c[k]), ptr(f, s->next[k]), shape_numel(&m->val[s->c[k]].sh));
			}
			if (s->tid >= 0) f->steps[s->tid] = s->T;
			break;
		}
		case CLS_THINK: {
			const tg_t *y = ptr(f, in->yield);
			tg_copy(o, ptr(f, in->init), n);
			tg_t sv = 65536;
			long long thr = to_fixed(in->eps, 16);
			if (!(thr > 0 || in->eps == 0)) thr = 1;
			int it;
			for (it = 0; it < in->maxit;) {
				block(f, in->body);
				it++;
				tg_t d = tg_delta(y, o, n);
				tg_copy(o, y, n);
				if (in->eps >= 0 && d <= thr) break;
				if (in->halt >= 0) {
					const tg_t *hp = ptr(f, in->halt);
					tg_t p = hp[0] < 0 ? 0 : hp[0] > 65536 ? 65536 : hp[0];
					sv = tg_fmul(sv, 65536 - p);
					if (65536 - sv > to_fixed(in->hthr, 16)) break;
				}
			}
			f->steps[in->tid] = it;
			break;
		}
		default: abort(); /* ops outside the quantized batch path */
		}
	}
}

void ref_fixed_run(const Module *m, const int *in, int *out, int *steps, int *arena)
{
	FX f = { m, (tg_t *)arena, (const tg_t *)in, steps };
	block(&f, &m->top);
	tg_copy((tg_t *)out, ptr(&f, m->output), shape_numel(&m->val[m->output].sh));
}
