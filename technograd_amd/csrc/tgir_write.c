/* The canonical TGIR writer for a module the backend read (tgm.h): the text
 * the reference's ir_write produces (src/ir.c:40-202) for the same module.
 * Named values keep their names; temporaries are numbered from the count of
 * named values, in the order a reader recreates them (pre-order: a think's
 * result before its body; a scan's carries, slices, body, then its stacks);
 * params and states in module order, float values as %.9g, eight per line;
 * quantized params as scales (eight per line) and one code per element
 * (24 per line). Used by tg_hip_quantize_model to write a quantized model. */
#include "tgm.h"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
	const tgm_module *m;
	char *s;
	size_t n, cap;
	int *ren, fail;
} W;

static void put(W *w, const char *fmt, ...)
{
	va_list ap;
	for (;;) {
		if (w->fail) return;
		va_start(ap, fmt);
		int k = vsnprintf(w->s + w->n, w->cap - w->n, fmt, ap);
		va_end(ap);
		if (k < 0) {
			w->fail = 1;
			return;
		}
		if ((size_t)k < w->cap - w->n) {
			w->n += (size_t)k;
			return;
		}
		size_t cap = 2 * w->cap + (size_t)k;
		char *s = realloc(w->s, cap);
		if (!s) {
			w->fail = 1;
			return;
		}
		w->s = s;
		w->cap = cap;
	}
}

static void indent(W *w, int d)
{
	for (int i = 0; i < d; i++) put(w, "  ");
}

static const char *shape(const tgm_shape *s, char *buf) /* 64 bytes */
{
	int o = snprintf(buf, 64, "(f32");
	for (int i = 0; i < s->rank && o < 64; i++) o += snprintf(buf + o, (size_t)(64 - o), " %d", s->dim[i]);
	if (o < 64) snprintf(buf + o, (size_t)(64 - o), ")");
	return buf;
}

static const char *vn(W *w, int v, char *buf) /* 64 bytes */
{
	if (w->m->val[v].name) snprintf(buf, 64, "%s", w->m->val[v].name);
	else snprintf(buf, 64, "%%%d", w->ren[v]);
	return buf;
}

static void number(W *w, const tgm_block *b, int *next)
{
	for (int i = 0; i < b->len; i++) {
		const tgm_ins *in = &b->v[i];
		if (in->op == TGM_SCAN) {
			for (int k = 0; k < in->nc; k++) w->ren[in->c[k]] = (*next)++;
			for (int j = 0; j < in->nx; j++) w->ren[in->xt[j]] = (*next)++;
			number(w, in->body, next);
			for (int y = 0; y < in->ny; y++) w->ren[in->ys[y]] = (*next)++;
			continue;
		}
		w->ren[in->out] = (*next)++;
		if (in->op == TGM_THINK) number(w, in->body, next);
	}
}

static void block(W *w, const tgm_block *b, int d)
{
	const tgm_module *m = w->m;
	char sh[64], n0[64], n1[64];
	for (int i = 0; i < b->len; i++) {
		const tgm_ins *in = &b->v[i];
		indent(w, d);
		if (in->op == TGM_SCAN) {
			put(w, "(scan %d %s%s\n", in->T, in->reverse ? "reverse" : "forward", in->stid >= 0 ? " steps" : "");
			for (int k = 0; k < in->nc; k++) {
				indent(w, d + 1);
				put(w, "(carry %s %s %s)\n", vn(w, in->c[k], n0), shape(&m->val[in->c[k]].sh, sh), vn(w, in->cinit[k], n1));
			}
			for (int j = 0; j < in->nx; j++) {
				indent(w, d + 1);
				put(w, "(in %s %s %s)\n", vn(w, in->xt[j], n0), shape(&m->val[in->xt[j]].sh, sh), vn(w, in->x[j], n1));
			}
			indent(w, d + 1);
			put(w, "(body\n");
			block(w, in->body, d + 2);
			indent(w, d + 1);
			put(w, ")\n");
			for (int k = 0; k < in->nc; k++) {
				indent(w, d + 1);
				put(w, "(next %s %s)\n", vn(w, in->c[k], n0), vn(w, in->cnext[k], n1));
			}
			for (int y = 0; y < in->ny; y++) {
				indent(w, d + 1);
				put(w, "(emit %s %s %s)\n", vn(w, in->ys[y], n0), shape(&m->val[in->ys[y]].sh, sh), vn(w, in->y[y], n1));
			}
			indent(w, d);
			put(w, ")\n");
			continue;
		}
		put(w, "(%s %s ", vn(w, in->out, n0), shape(&m->val[in->out].sh, sh));
		if (in->op == TGM_CONST) {
			put(w, "(const %.9g))\n", (double)in->k);
		} else if (in->op == TGM_THINK) {
			put(w, "(think %s %d ", vn(w, in->init, n1), in->maxit);
			if (in->eps < 0) put(w, "none\n");
			else put(w, "%.9g\n", (double)in->eps);
			block(w, in->body, d + 1);
			indent(w, d + 1);
			put(w, "(yield %s)", vn(w, in->yield, n1));
			if (in->halt >= 0) {
				put(w, "\n");
				indent(w, d + 1);
				put(w, "(halt %s %.9g)", vn(w, in->halt, n1), (double)in->hthr);
			}
			put(w, "))\n");
		} else {
			put(w, "(%s", tgm_op_name(in->op));
			for (int j = 0; j < in->na; j++) put(w, " %s", vn(w, in->a[j], n1));
			put(w, "))\n");
		}
	}
}

char *tgm_write(const tgm_module *m)
{
	W w = { m, malloc(1 << 16), 0, 1 << 16, calloc((size_t)(m->nval ? m->nval : 1), sizeof(int)), 0 };
	if (!w.s || !w.ren || m->nupd) { /* state updates are not recorded by the reader */
		free(w.s);
		free(w.ren);
		return NULL;
	}
	char sh[64], n0[64];
	int next = 0;
	for (int v = 0; v < m->nval; v++)
		if (m->val[v].kind != TGM_TMP) next++;
	number(&w, &m->top, &next);
	put(&w, "(tgir 1\n  (model %s)\n", m->name);
	for (int v = 0; v < m->nval; v++) {
		const tgm_value *x = &m->val[v];
		if (x->kind != TGM_PARAM && x->kind != TGM_STATE) continue;
		if (x->qbits) {
			int nch = x->sh.dim[x->qaxis];
			put(&w, "  (param %s %s\n    (quant %d %d\n      (scale", x->name, shape(&x->sh, sh), x->qbits, x->qaxis);
			for (int i = 0; i < nch; i++) put(&w, "%s %.9g", i && i % 8 == 0 ? "\n            " : "", (double)x->qs[i]);
			put(&w, ")\n      (codes");
			for (long i = 0; i < x->n; i++) put(&w, "%s %d", i && i % 24 == 0 ? "\n            " : "", tgm_code(x, i));
			put(&w, ")))\n");
			continue;
		}
		put(&w, "  (%s %s %s\n    (data", x->kind == TGM_STATE ? "state" : "param", x->name, shape(&x->sh, sh));
		for (long i = 0; i < x->n; i++) {
			if (i && i % 8 == 0) put(&w, "\n         ");
			put(&w, " %.9g", (double)x->data[i]);
		}
		put(&w, "))\n");
	}
	for (int i = 0; i < m->ninputs; i++) {
		const tgm_value *x = &m->val[m->inputs[i]];
		put(&w, "  (input %s %s)\n", x->name, shape(&x->sh, sh));
	}
	put(&w, "  (block\n");
	block(&w, &m->top, 2);
	put(&w, "  )\n  (output %s))\n", vn(&w, m->output, n0));
	free(w.ren);
	if (w.fail) {
		free(w.s);
		return NULL;
	}
	return w.s;
}
