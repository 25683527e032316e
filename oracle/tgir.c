/* TEST INFRASTRUCTURE ONLY — oracle TGIR reader and writer.
 *
 * Restates the TGIR grammar and reader of the reference (src/ir.c:1-24
 * grammar, :458-554 ir_read, :258-350 scan, :352-456 block/think) and its
 * S-expression atoms (src/sexp.c:112-126: a token is a number when strtod
 * consumes it whole and it starts with a digit, or with + - . and is longer
 * than one character). Quantized params follow src/ir.c:478-509: one scale per
 * channel, one code per element, codes range-checked (+-127 / +-7), int4 codes
 * packed low nibble first, and `data` keeps code * scale in f32.
 *
 * The writer restates src/ir.c:150-202 (canonical numbering of temporaries,
 * "%.9g" numbers, 8 scales / 24 codes / 8 data values per line).
 *
 * Pinned by: tests/golden (files written by the reference's own ir_write are
 * read back and re-written byte-identically; quantized files read here and run
 * through the oracle VM match the reference VM byte for byte). */
#include "tgo.h"

#include <ctype.h>
#include <math.h>
#include <setjmp.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
	const char *p;
	int line;
	jmp_buf jb;
	char *err;
	int errn;
	tgo_module *m;
	/* scope: a stack of (name, value) pairs */
	char **names;
	int *vals, n, cap;
} P;

static void fail(P *r, const char *fmt, ...)
{
	va_list ap;
	va_start(ap, fmt);
	int k = snprintf(r->err, (size_t)r->errn, "line %d: ", r->line);
	if (k > 0 && k < r->errn) vsnprintf(r->err + k, (size_t)(r->errn - k), fmt, ap);
	va_end(ap);
	longjmp(r->jb, 1);
}

static void *xcalloc(P *r, size_t n, size_t s)
{
	void *p = calloc(n ? n : 1, s ? s : 1);
	if (!p) fail(r, "out of memory");
	return p;
}

static void skip(P *r)
{
	for (;;) {
		while (isspace((unsigned char)*r->p)) {
			if (*r->p == '\n') r->line++;
			r->p++;
		}
		if (*r->p != ';') return;
		while (*r->p && *r->p != '\n') r->p++;
	}
}

static int peek(P *r)
{
	skip(r);
	return *r->p;
}

static void open_(P *r)
{
	if (peek(r) != '(') fail(r, "expected '('");
	r->p++;
}

static void close_(P *r)
{
	if (peek(r) != ')') fail(r, "expected ')'");
	r->p++;
}

/* An atom: returns its text in buf; *isnum and *num say whether it is a number. */
static void atom(P *r, char *buf, size_t bn, int *isnum, double *num)
{
	skip(r);
	const char *s = r->p;
	if (!*s || *s == '(' || *s == ')') fail(r, "expected an atom");
	while (*r->p && !isspace((unsigned char)*r->p) && *r->p != '(' && *r->p != ')' && *r->p != ';' && *r->p != '"') r->p++;
	size_t n = (size_t)(r->p - s);
	if (n >= bn) fail(r, "atom too long");
	memcpy(buf, s, n);
	buf[n] = 0;
	char *end;
	double d = strtod(buf, &end);
	*isnum = *end == 0 && (isdigit((unsigned char)buf[0]) || ((buf[0] == '-' || buf[0] == '+' || buf[0] == '.') && n > 1));
	*num = d;
}

static double number(P *r, const char *what)
{
	char b[128];
	int isn;
	double d;
	atom(r, b, sizeof b, &isn, &d);
	if (!isn) fail(r, "expected a number (%s), got '%s'", what, b);
	return d;
}

static void symbol(P *r, char *buf, size_t bn)
{
	int isn;
	double d;
	atom(r, buf, bn, &isn, &d);
	if (isn) fail(r, "expected a name, got '%s'", buf);
}

/* the next token is '(' followed by the symbol s */
static int peek_head(P *r, const char *s)
{
	if (peek(r) != '(') return 0;
	const char *q = r->p + 1;
	while (isspace((unsigned char)*q)) q++;
	size_t n = strlen(s);
	return strncmp(q, s, n) == 0 && (isspace((unsigned char)q[n]) || q[n] == ')' || q[n] == '(');
}

static tgo_shape shape(P *r)
{
	tgo_shape s = { 0 };
	char b[64];
	open_(r);
	symbol(r, b, sizeof b);
	if (strcmp(b, "f32")) fail(r, "expected type (f32 d...)");
	while (peek(r) != ')') {
		if (s.rank == TGO_MAXRANK) fail(r, "rank exceeds %d", TGO_MAXRANK);
		double d = number(r, "dimension");
		if (d < 1 || d != (double)(int)d) fail(r, "bad dimension");
		s.dim[s.rank++] = (int)d;
	}
	close_(r);
	return s;
}

int tgo_numel(const tgo_shape *s)
{
	int n = 1;
	for (int i = 0; i < s->rank; i++) n *= s->dim[i];
	return n;
}

static int shape_eq(const tgo_shape *a, const tgo_shape *b)
{
	if (a->rank != b->rank) return 0;
	for (int i = 0; i < a->rank; i++)
		if (a->dim[i] != b->dim[i]) return 0;
	return 1;
}

static int new_value(P *r, int kind, const tgo_shape *sh, const char *name)
{
	tgo_module *m = r->m;
	if (m->nval == m->capval) {
		m->capval = m->capval ? 2 * m->capval : 64;
		m->val = realloc(m->val, (size_t)m->capval * sizeof *m->val);
		if (!m->val) fail(r, "out of memory");
	}
	tgo_value *v = &m->val[m->nval];
	memset(v, 0, sizeof *v);
	v->kind = kind;
	v->sh = *sh;
	v->n = tgo_numel(sh);
	v->off = -1;
	if (name) v->name = strdup(name);
	return m->nval++;
}

static int get(P *r, const char *name)
{
	for (int i = r->n - 1; i >= 0; i--)
		if (!strcmp(r->names[i], name)) return r->vals[i];
	fail(r, "undefined value '%s'", name);
	return -1;
}

static int get_next(P *r)
{
	char b[128];
	symbol(r, b, sizeof b);
	return get(r, b);
}

static void def(P *r, const char *name, int v)
{
	for (int i = 0; i < r->n; i++)
		if (!strcmp(r->names[i], name)) fail(r, "redefinition of '%s'", name);
	if (r->n == r->cap) {
		r->cap = r->cap ? 2 * r->cap : 64;
		r->names = realloc(r->names, (size_t)r->cap * sizeof *r->names);
		r->vals = realloc(r->vals, (size_t)r->cap * sizeof *r->vals);
	}
	r->names[r->n] = strdup(name);
	r->vals[r->n++] = v;
}

static void drop_to(P *r, int mark)
{
	while (r->n > mark) free(r->names[--r->n]);
}

static tgo_ins *push(P *r, tgo_block *b)
{
	if (b->len == b->cap) {
		b->cap = b->cap ? 2 * b->cap : 8;
		b->v = realloc(b->v, (size_t)b->cap * sizeof *b->v);
		if (!b->v) fail(r, "out of memory");
	}
	tgo_ins *in = &b->v[b->len++];
	memset(in, 0, sizeof *in);
	in->init = in->yield = in->halt = in->tid = in->stid = -1;
	for (int j = 0; j < TGO_MAXARGS; j++) in->a[j] = -1;
	return in;
}

static const struct {
	const char *name;
	int op, arity;
} optab[] = {
	{ "add", O_ADD, 2 }, { "sub", O_SUB, 2 }, { "mul", O_MUL, 2 }, { "div", O_DIV, 2 }, { "max", O_MAX, 2 }, { "min", O_MIN, 2 },
	{ "neg", O_NEG, 1 }, { "tanh", O_TANH, 1 }, { "relu", O_RELU, 1 }, { "sigmoid", O_SIGMOID, 1 }, { "exp", O_EXP, 1 },
	{ "sqrt", O_SQRT, 1 }, { "gelu", O_GELU, 1 }, { "silu", O_SILU, 1 }, { "softplus", O_SOFTPLUS, 1 }, { "log", O_LOG, 1 },
	{ "sin", O_SIN, 1 }, { "cos", O_COS, 1 }, { "floor", O_FLOOR, 1 }, { "step", O_STEP, 1 }, { "matmul", O_MATMUL, 2 },
	{ "softmax", O_SOFTMAX, 1 }, { "rmsnorm", O_RMSNORM, 1 }, { "sum", O_SUM, 1 }, { "mean", O_MEAN, 1 },
	{ "transpose", O_TRANSPOSE, 1 }, { "outer", O_OUTER, 2 }, { "reshape", O_RESHAPE, 1 }, { "take", O_TAKE, 2 },
};

static const char *op_name(int op)
{
	if (op == O_CONST) return "const";
	for (size_t i = 0; i < sizeof optab / sizeof optab[0]; i++)
		if (optab[i].op == op) return optab[i].name;
	return "?";
}

static void block_items(P *r, tgo_block *b, int stop_at_yield);

/* (scan T forward|reverse [steps] (carry ..)... (in ..)... (body ...) (next ..)... (emit ..)...)
 * Scoping as src/ir.c:258-350. */
static void scan_item(P *r, tgo_block *b)
{
	char s[128], nm[128];
	symbol(r, s, sizeof s); /* "scan" */
	double T = number(r, "scan steps");
	if (T < 1 || T != (double)(int)T) fail(r, "malformed scan (steps)");
	symbol(r, s, sizeof s);
	if (strcmp(s, "forward") && strcmp(s, "reverse")) fail(r, "malformed scan (direction)");
	int reverse = !strcmp(s, "reverse"), stid = -1;
	if (peek(r) != '(') {
		symbol(r, s, sizeof s);
		if (strcmp(s, "steps")) fail(r, "malformed scan");
		stid = r->m->nthink++;
	}
	int cap = 16, nc = 0, nx = 0, ny = 0;
	int *c = xcalloc(r, (size_t)cap, sizeof *c), *ci = xcalloc(r, (size_t)cap, sizeof *ci);
	char **cn = xcalloc(r, (size_t)cap, sizeof *cn), **xn = xcalloc(r, (size_t)cap, sizeof *xn), **yn = xcalloc(r, (size_t)cap, sizeof *yn);
	int *x = xcalloc(r, (size_t)cap, sizeof *x), *xt = xcalloc(r, (size_t)cap, sizeof *xt);
	while (peek_head(r, "carry")) {
		if (nc == cap) fail(r, "too many scan carries");
		open_(r);
		symbol(r, s, sizeof s);
		symbol(r, nm, sizeof nm);
		tgo_shape sh = shape(r);
		int init = get_next(r);
		close_(r);
		if (!shape_eq(&sh, &r->m->val[init].sh)) fail(r, "carry type differs from its initial value");
		cn[nc] = strdup(nm);
		ci[nc] = init;
		c[nc++] = new_value(r, TGO_TMP, &sh, NULL);
	}
	if (!nc) fail(r, "malformed scan (needs a carry)");
	while (peek_head(r, "in")) {
		if (nx == cap) fail(r, "too many scan sequences");
		open_(r);
		symbol(r, s, sizeof s);
		symbol(r, nm, sizeof nm);
		tgo_shape sh = shape(r);
		int q = get_next(r);
		close_(r);
		tgo_shape want = r->m->val[q].sh;
		if (want.rank < 1 || want.dim[0] != (int)T) fail(r, "sequence does not have %d steps along its first axis", (int)T);
		for (int d = 1; d < want.rank; d++) want.dim[d - 1] = want.dim[d];
		want.rank--;
		if (!shape_eq(&sh, &want)) fail(r, "slice type differs from a row of its sequence");
		xn[nx] = strdup(nm);
		x[nx] = q;
		xt[nx++] = new_value(r, TGO_TMP, &sh, NULL);
	}
	int mark = r->n;
	for (int k = 0; k < nc; k++) def(r, cn[k], c[k]);
	for (int j = 0; j < nx; j++) def(r, xn[j], xt[j]);
	if (!peek_head(r, "body")) fail(r, "malformed scan (body)");
	int idx = b->len;
	push(r, b);
	tgo_block *body = xcalloc(r, 1, sizeof *body);
	open_(r);
	symbol(r, s, sizeof s);
	block_items(r, body, 0);
	close_(r);
	int *nxt = xcalloc(r, (size_t)nc, sizeof *nxt);
	for (int k = 0; k < nc; k++) {
		if (!peek_head(r, "next")) fail(r, "malformed scan (next)");
		open_(r);
		symbol(r, s, sizeof s);
		if (get_next(r) != c[k]) fail(r, "'next' entries must follow the carries in order");
		int nv = get_next(r);
		close_(r);
		if (!shape_eq(&r->m->val[nv].sh, &r->m->val[c[k]].sh)) fail(r, "next value shape differs from its carry");
		nxt[k] = nv;
	}
	int *yv = xcalloc(r, (size_t)cap, sizeof *yv);
	tgo_shape ysh[16];
	while (peek(r) == '(') {
		if (!peek_head(r, "emit") || ny == cap) fail(r, "malformed scan (emit)");
		open_(r);
		symbol(r, s, sizeof s);
		symbol(r, nm, sizeof nm);
		tgo_shape sh = shape(r);
		int v = get_next(r);
		close_(r);
		tgo_shape want = r->m->val[v].sh;
		if (want.rank == TGO_MAXRANK) fail(r, "stack rank exceeds %d", TGO_MAXRANK);
		for (int d = want.rank; d > 0; d--) want.dim[d] = want.dim[d - 1];
		want.dim[0] = (int)T;
		want.rank++;
		if (!shape_eq(&sh, &want)) fail(r, "emit type differs from the stack of its value");
		yn[ny] = strdup(nm);
		ysh[ny] = sh;
		yv[ny++] = v;
	}
	drop_to(r, mark);
	for (int k = 0; k < nc; k++) def(r, cn[k], c[k]);
	int *ys = xcalloc(r, (size_t)(ny ? ny : 1), sizeof *ys);
	for (int y = 0; y < ny; y++) {
		ys[y] = new_value(r, TGO_TMP, &ysh[y], NULL);
		def(r, yn[y], ys[y]);
	}
	tgo_ins *in = &b->v[idx];
	in->op = O_SCAN;
	in->T = (int)T;
	in->reverse = reverse;
	in->stid = stid;
	in->nc = nc;
	in->c = c;
	in->cinit = ci;
	in->cnext = nxt;
	in->nx = nx;
	in->x = x;
	in->xt = xt;
	in->ny = ny;
	in->y = yv;
	in->ys = ys;
	in->body = body;
	in->out = c[0];
	for (int k = 0; k < nc; k++) free(cn[k]);
	for (int j = 0; j < nx; j++) free(xn[j]);
	for (int y = 0; y < ny; y++) free(yn[y]);
	free(cn);
	free(xn);
	free(yn);
}

/* Items of a block until ')' (or, in a think body, until the (yield ..) form). */
static void block_items(P *r, tgo_block *b, int stop_at_yield)
{
	char s[128], nm[128];
	for (;;) {
		if (peek(r) == ')') return;
		if (stop_at_yield && peek_head(r, "yield")) return;
		open_(r);
		skip(r);
		if (!strncmp(r->p, "scan", 4) && isspace((unsigned char)r->p[4])) { /* a list headed by the symbol scan */
			scan_item(r, b);
			close_(r);
			continue;
		}
		symbol(r, nm, sizeof nm);
		tgo_shape decl = shape(r);
		open_(r);
		symbol(r, s, sizeof s);
		int out;
		if (!strcmp(s, "const")) {
			double k = number(r, "const");
			close_(r);
			out = new_value(r, TGO_TMP, &decl, NULL);
			tgo_ins *in = push(r, b);
			in->op = O_CONST;
			in->k = (float)k;
			in->out = out;
		} else if (!strcmp(s, "think")) {
			int init = get_next(r);
			double mx = number(r, "think budget");
			if (mx < 1) fail(r, "malformed think budget");
			double eps = -1;
			char e[64];
			int isn;
			atom(r, e, sizeof e, &isn, &eps);
			if (!isn) {
				if (strcmp(e, "none")) fail(r, "malformed think threshold");
				eps = -1;
			} else if (eps < 0) fail(r, "malformed think threshold");
			if (!shape_eq(&decl, &r->m->val[init].sh)) fail(r, "declared shape differs from the think state");
			out = new_value(r, TGO_TMP, &decl, NULL);
			int idx = b->len;
			push(r, b);
			int tid = r->m->nthink++;
			tgo_block *body = xcalloc(r, 1, sizeof *body);
			int mark = r->n;
			def(r, nm, out); /* the state is visible in the body */
			block_items(r, body, 1);
			if (!peek_head(r, "yield")) fail(r, "think (missing yield)");
			open_(r);
			symbol(r, s, sizeof s);
			int y = get_next(r);
			close_(r);
			int halt = -1;
			double thr = 0;
			if (peek_head(r, "halt")) {
				open_(r);
				symbol(r, s, sizeof s);
				halt = get_next(r);
				thr = number(r, "halt threshold");
				close_(r);
				if (!(thr > 0 && thr < 1) || eps >= 0) fail(r, "think halt (value, threshold in (0, 1); no until)");
				if (r->m->val[halt].sh.rank != 0) fail(r, "halting value must be a scalar");
			}
			close_(r);
			if (!shape_eq(&r->m->val[y].sh, &decl)) fail(r, "yield shape differs from state shape");
			drop_to(r, mark);
			tgo_ins *in = &b->v[idx];
			in->op = O_THINK;
			in->out = out;
			in->init = init;
			in->maxit = (int)mx;
			in->eps = eps < 0 ? -1.0f : (float)eps;
			in->tid = tid;
			in->body = body;
			in->yield = y;
			in->halt = halt;
			in->hthr = (float)thr;
		} else {
			int op = -1, ar = 0;
			for (size_t i = 0; i < sizeof optab / sizeof optab[0]; i++)
				if (!strcmp(optab[i].name, s)) {
					op = optab[i].op;
					ar = optab[i].arity;
				}
			if (op < 0) fail(r, "unknown or unsupported op '%s'", s);
			int a[TGO_MAXARGS], na = 0;
			while (peek(r) != ')') {
				if (na == TGO_MAXARGS) fail(r, "too many operands");
				a[na++] = get_next(r);
			}
			close_(r);
			if (na != ar) fail(r, "'%s' takes %d operand(s), got %d", s, ar, na);
			if (op == O_RESHAPE && r->m->val[a[0]].n != tgo_numel(&decl)) fail(r, "reshape changes the element count");
			out = new_value(r, TGO_TMP, &decl, NULL);
			tgo_ins *in = push(r, b);
			in->op = op;
			in->out = out;
			in->na = na;
			for (int j = 0; j < na; j++) in->a[j] = a[j];
		}
		close_(r);
		def(r, nm, out);
	}
}

static void set_code(tgo_value *x, long j, int c)
{
	if (x->qbits == 8) {
		x->q[j] = (signed char)c;
		return;
	}
	unsigned char b = (unsigned char)x->q[j / 2];
	b = j % 2 ? (unsigned char)((b & 0x0f) | (unsigned char)((unsigned)c << 4)) : (unsigned char)((b & 0xf0) | (c & 0x0f));
	x->q[j / 2] = (signed char)b;
}

/* Test-only extension of the reader (the reference reads text only): a
 * param's values from a raw little-endian file next to the text, for models
 * too large to write as text: `(data-file PATH)` (f32), and inside `quant`
 * `(scale-file PATH)` (f32, one per channel) and `(codes-file PATH)` (int8,
 * one per element). The values are the ones the text forms would give. */
static void raw_file(P *r, void *dst, size_t bytes)
{
	char path[4096];
	int isn;
	double d;
	atom(r, path, sizeof path, &isn, &d);
	FILE *f = fopen(path, "rb");
	if (!f) fail(r, "cannot open '%s'", path);
	const size_t got = fread(dst, 1, bytes, f);
	const int extra = fgetc(f) != EOF;
	fclose(f);
	if (got != bytes || extra) fail(r, "'%s' does not hold %zu bytes", path, bytes);
}

static void top_form(P *r, int *seen_block, int *seen_out)
{
	char h[64], nm[128], s[64];
	tgo_module *m = r->m;
	open_(r);
	symbol(r, h, sizeof h);
	if (!strcmp(h, "model")) {
		symbol(r, nm, sizeof nm);
		if (m->name) fail(r, "malformed model");
		m->name = strdup(nm);
		close_(r);
		return;
	}
	if (!m->name) fail(r, "(model ...) must come first");
	if (!strcmp(h, "param") || !strcmp(h, "state")) {
		if (*seen_block) fail(r, "malformed %s", h);
		symbol(r, nm, sizeof nm);
		tgo_shape sh = shape(r);
		int kind = strcmp(h, "state") ? TGO_PARAM : TGO_STATE;
		int v = new_value(r, kind, &sh, nm);
		tgo_value *x = &m->val[v];
		open_(r);
		symbol(r, s, sizeof s);
		if (!strcmp(s, "quant") && kind == TGO_PARAM) {
			double bits = number(r, "quant bits"), axis = number(r, "quant axis");
			if (bits != 8 && bits != 4) fail(r, "malformed quant bits (8 or 4)");
			if ((axis != 0 && axis != 1) || sh.rank != 2) fail(r, "malformed quant axis (0 or 1, rank-2 param)");
			x = &m->val[v];
			x->qbits = (int)bits;
			x->qaxis = (int)axis;
			int nch = sh.dim[x->qaxis];
			x->qs = xcalloc(r, (size_t)nch, sizeof(float));
			x->q = xcalloc(r, (size_t)(x->qbits == 8 ? x->n : (x->n + 1) / 2), 1);
			x->data = xcalloc(r, (size_t)x->n, sizeof(float));
			open_(r);
			symbol(r, s, sizeof s);
			if (!strcmp(s, "scale-file")) {
				raw_file(r, x->qs, (size_t)nch * sizeof(float));
			} else {
				if (strcmp(s, "scale")) fail(r, "malformed quant scales");
				for (int j = 0; j < nch; j++) {
					if (peek(r) == ')') fail(r, "malformed quant scales (one per channel)");
					x->qs[j] = (float)number(r, "scale");
				}
			}
			close_(r);
			open_(r);
			symbol(r, s, sizeof s);
			int lim = x->qbits == 8 ? 127 : 7;
			signed char *raw = NULL;
			if (!strcmp(s, "codes-file")) {
				raw = xcalloc(r, (size_t)x->n, 1);
				raw_file(r, raw, (size_t)x->n);
			} else if (strcmp(s, "codes")) {
				fail(r, "malformed quant codes");
			}
			for (long j = 0; j < x->n; j++) {
				double c;
				if (raw) {
					c = raw[j];
				} else {
					if (peek(r) == ')') fail(r, "malformed quant codes (one per element)");
					c = number(r, "code");
				}
				if (c != (double)(int)c || fabs(c) > lim) fail(r, "malformed code");
				set_code(x, j, (int)c);
				long ch = x->qaxis == 0 ? j / sh.dim[1] : j % sh.dim[1];
				x->data[j] = (float)(int)c * x->qs[ch];
			}
			free(raw);
			close_(r);
			close_(r);
		} else if (!strcmp(s, "data-file")) {
			x->data = xcalloc(r, (size_t)x->n, sizeof(float));
			raw_file(r, x->data, (size_t)x->n * sizeof(float));
			close_(r);
		} else if (!strcmp(s, "data")) {
			x->data = xcalloc(r, (size_t)x->n, sizeof(float));
			long j = 0;
			while (peek(r) != ')') {
				double d = number(r, "data");
				if (j < x->n) x->data[j] = (float)d;
				j++;
			}
			if (j != x->n) fail(r, "param '%s' needs %d values, has %ld", nm, x->n, j);
			close_(r);
		} else {
			fail(r, "malformed %s", h);
		}
		close_(r);
		def(r, nm, v);
		return;
	}
	if (!strcmp(h, "input")) {
		if (*seen_block) fail(r, "malformed input");
		symbol(r, nm, sizeof nm);
		tgo_shape sh = shape(r);
		close_(r);
		int v = new_value(r, TGO_INPUT, &sh, nm);
		m->val[v].index = m->ninputs;
		m->inputs = realloc(m->inputs, (size_t)(m->ninputs + 1) * sizeof *m->inputs);
		m->inputs[m->ninputs++] = v;
		def(r, nm, v);
		return;
	}
	if (!strcmp(h, "block")) {
		if (*seen_block) fail(r, "malformed block (duplicate)");
		*seen_block = 1;
		block_items(r, &m->top, 0);
		close_(r);
		return;
	}
	if (!strcmp(h, "update")) {
		if (!*seen_block) fail(r, "malformed update");
		int depth = 1;
		while (depth) { /* state updates are recorded only to refuse the model */
			int c = peek(r);
			if (!c) fail(r, "unterminated update");
			if (c == '(') depth++;
			if (c == ')') depth--;
			r->p++;
		}
		m->nupd++;
		return;
	}
	if (!strcmp(h, "output")) {
		if (!*seen_block || *seen_out) fail(r, "malformed output");
		*seen_out = 1;
		m->output = get_next(r);
		close_(r);
		return;
	}
	fail(r, "unknown top-level form '%s'", h);
}

static void plan_arena(tgo_module *m)
{
	long off = 0;
	for (int v = 0; v < m->nval; v++)
		if (m->val[v].kind == TGO_TMP) {
			m->val[v].off = off;
			off += (m->val[v].n + 3) / 4 * 4;
		}
	m->arena = off ? off : 1;
	m->per = 0;
	for (int i = 0; i < m->ninputs; i++) m->per += m->val[m->inputs[i]].n;
	m->nout = m->val[m->output].n;
}

tgo_module *tgo_load(const char *text, char *err, int errn)
{
	P r;
	memset(&r, 0, sizeof r);
	r.p = text;
	r.line = 1;
	r.err = err;
	r.errn = errn;
	r.m = calloc(1, sizeof *r.m);
	if (!r.m) return NULL;
	r.m->output = -1;
	if (setjmp(r.jb)) {
		drop_to(&r, 0);
		free(r.names);
		free(r.vals);
		tgo_free(r.m);
		return NULL;
	}
	int seen_block = 0, seen_out = 0;
	open_(&r);
	char s[64];
	symbol(&r, s, sizeof s);
	if (strcmp(s, "tgir")) fail(&r, "expected (tgir 1 ...)");
	if (number(&r, "version") != 1) fail(&r, "unsupported TGIR version");
	while (peek(&r) != ')') top_form(&r, &seen_block, &seen_out);
	close_(&r);
	if (peek(&r)) fail(&r, "expected exactly one (tgir ...) form");
	if (!r.m->name) fail(&r, "missing (model ...)");
	if (!r.m->ninputs) fail(&r, "module has no inputs");
	if (!seen_out) fail(&r, "missing (output ...)");
	drop_to(&r, 0);
	free(r.names);
	free(r.vals);
	plan_arena(r.m);
	return r.m;
}

static void free_block(tgo_block *b)
{
	for (int i = 0; i < b->len; i++) {
		tgo_ins *in = &b->v[i];
		if (in->body) {
			free_block(in->body);
			free(in->body);
		}
		if (in->op == O_SCAN) {
			free(in->c);
			free(in->cinit);
			free(in->cnext);
			free(in->x);
			free(in->xt);
			free(in->y);
			free(in->ys);
		}
	}
	free(b->v);
}

void tgo_free(tgo_module *m)
{
	if (!m) return;
	for (int v = 0; v < m->nval; v++) {
		tgo_value *x = &m->val[v];
		free(x->name);
		free(x->data);
		free(x->d64);
		free(x->q);
		free(x->qs);
		free(x->fx);
		free(x->fqs);
	}
	free(m->val);
	free(m->inputs);
	free_block(&m->top);
	free(m->name);
	free(m);
}

int tgo_info(const tgo_module *m, int *per, int *nout, int *nthink, long *arena)
{
	*per = m->per;
	*nout = m->nout;
	*nthink = m->nthink;
	*arena = m->arena;
	return m->nupd;
}

int tgo_qget(const signed char *q, int bits, long i)
{
	if (bits == 8) return q[i];
	int b = q[i >> 1];
	return (i & 1) ? (b >> 4) : (int)(signed char)(unsigned char)((unsigned)b << 4) >> 4;
}

/* ---- writer (src/ir.c:150-202) ---- */

typedef struct {
	char *s;
	size_t n, cap;
} Buf;

static void put(Buf *b, const char *fmt, ...)
{
	va_list ap;
	for (;;) {
		va_start(ap, fmt);
		int k = vsnprintf(b->s + b->n, b->cap - b->n, fmt, ap);
		va_end(ap);
		if (k >= 0 && (size_t)k < b->cap - b->n) {
			b->n += (size_t)k;
			return;
		}
		b->cap = b->cap * 2 + (size_t)(k > 0 ? k : 0) + 256;
		b->s = realloc(b->s, b->cap);
	}
}

static void number_vals(const tgo_module *m, const tgo_block *b, int *ren, int *next)
{
	for (int i = 0; i < b->len; i++) {
		const tgo_ins *in = &b->v[i];
		if (in->op == O_SCAN) {
			for (int k = 0; k < in->nc; k++) ren[in->c[k]] = (*next)++;
			for (int j = 0; j < in->nx; j++) ren[in->xt[j]] = (*next)++;
			number_vals(m, in->body, ren, next);
			for (int y = 0; y < in->ny; y++) ren[in->ys[y]] = (*next)++;
			continue;
		}
		ren[in->out] = (*next)++;
		if (in->op == O_THINK) number_vals(m, in->body, ren, next);
	}
}

static const char *vn(const tgo_module *m, const int *ren, int v, char *buf)
{
	if (m->val[v].name) return m->val[v].name;
	sprintf(buf, "%%%d", ren[v]);
	return buf;
}

static void shape_str(const tgo_shape *s, char *buf)
{
	int o = sprintf(buf, "(f32");
	for (int i = 0; i < s->rank; i++) o += sprintf(buf + o, " %d", s->dim[i]);
	sprintf(buf + o, ")");
}

static void indent(Buf *b, int d)
{
	for (int i = 0; i < d; i++) put(b, "  ");
}

static void write_block(const tgo_module *m, const tgo_block *bl, const int *ren, Buf *b, int d)
{
	char sh[96], n0[64], n1[64], n2[64];
	for (int i = 0; i < bl->len; i++) {
		const tgo_ins *in = &bl->v[i];
		indent(b, d);
		if (in->op == O_SCAN) {
			put(b, "(scan %d %s%s\n", in->T, in->reverse ? "reverse" : "forward", in->stid >= 0 ? " steps" : "");
			for (int k = 0; k < in->nc; k++) {
				shape_str(&m->val[in->c[k]].sh, sh);
				indent(b, d + 1);
				put(b, "(carry %s %s %s)\n", vn(m, ren, in->c[k], n0), sh, vn(m, ren, in->cinit[k], n1));
			}
			for (int j = 0; j < in->nx; j++) {
				shape_str(&m->val[in->xt[j]].sh, sh);
				indent(b, d + 1);
				put(b, "(in %s %s %s)\n", vn(m, ren, in->xt[j], n0), sh, vn(m, ren, in->x[j], n1));
			}
			indent(b, d + 1);
			put(b, "(body\n");
			write_block(m, in->body, ren, b, d + 2);
			indent(b, d + 1);
			put(b, ")\n");
			for (int k = 0; k < in->nc; k++) {
				indent(b, d + 1);
				put(b, "(next %s %s)\n", vn(m, ren, in->c[k], n0), vn(m, ren, in->cnext[k], n1));
			}
			for (int y = 0; y < in->ny; y++) {
				shape_str(&m->val[in->ys[y]].sh, sh);
				indent(b, d + 1);
				put(b, "(emit %s %s %s)\n", vn(m, ren, in->ys[y], n0), sh, vn(m, ren, in->y[y], n1));
			}
			indent(b, d);
			put(b, ")\n");
			continue;
		}
		shape_str(&m->val[in->out].sh, sh);
		put(b, "(%s %s ", vn(m, ren, in->out, n0), sh);
		if (in->op == O_CONST) {
			put(b, "(const %.9g))\n", (double)in->k);
		} else if (in->op == O_THINK) {
			put(b, "(think %s %d ", vn(m, ren, in->init, n1), in->maxit);
			if (in->eps < 0) put(b, "none\n");
			else put(b, "%.9g\n", (double)in->eps);
			write_block(m, in->body, ren, b, d + 1);
			indent(b, d + 1);
			put(b, "(yield %s)", vn(m, ren, in->yield, n2));
			if (in->halt >= 0) {
				put(b, "\n");
				indent(b, d + 1);
				put(b, "(halt %s %.9g)", vn(m, ren, in->halt, n2), (double)in->hthr);
			}
			put(b, "))\n");
		} else {
			put(b, "(%s", op_name(in->op));
			for (int j = 0; j < in->na; j++) put(b, " %s", vn(m, ren, in->a[j], n1));
			put(b, "))\n");
		}
	}
}

char *tgo_write(const tgo_module *m)
{
	Buf b = { malloc(1 << 16), 0, 1 << 16 };
	int *ren = calloc((size_t)(m->nval ? m->nval : 1), sizeof *ren), next = 0;
	char sh[96], n[64];
	for (int v = 0; v < m->nval; v++)
		if (m->val[v].kind != TGO_TMP) next++;
	number_vals(m, &m->top, ren, &next);
	put(&b, "(tgir 1\n  (model %s)\n", m->name);
	for (int v = 0; v < m->nval; v++) {
		const tgo_value *x = &m->val[v];
		if (x->kind != TGO_PARAM && x->kind != TGO_STATE) continue;
		shape_str(&x->sh, sh);
		if (x->qbits) {
			int nch = x->sh.dim[x->qaxis];
			put(&b, "  (param %s %s\n    (quant %d %d\n      (scale", x->name, sh, x->qbits, x->qaxis);
			for (int i = 0; i < nch; i++) put(&b, "%s %.9g", i && i % 8 == 0 ? "\n            " : "", (double)x->qs[i]);
			put(&b, ")\n      (codes");
			for (long i = 0; i < x->n; i++) put(&b, "%s %d", i && i % 24 == 0 ? "\n            " : "", tgo_qget(x->q, x->qbits, i));
			put(&b, ")))\n");
			continue;
		}
		put(&b, "  (%s %s %s\n    (data", x->kind == TGO_STATE ? "state" : "param", x->name, sh);
		for (long i = 0; i < x->n; i++) {
			if (i && i % 8 == 0) put(&b, "\n         ");
			put(&b, " %.9g", (double)x->data[i]);
		}
		put(&b, "))\n");
	}
	for (int i = 0; i < m->ninputs; i++) {
		const tgo_value *x = &m->val[m->inputs[i]];
		shape_str(&x->sh, sh);
		put(&b, "  (input %s %s)\n", x->name, sh);
	}
	put(&b, "  (block\n");
	write_block(m, &m->top, ren, &b, 2);
	put(&b, "  )\n  (output %s))\n", vn(m, ren, m->output, n));
	free(ren);
	return b.s;
}

void tgo_str_free(char *s) { free(s); }
