/* TGIR reader for the MI355X batch backend.
 *
 * Accepts the reference's canonical model text (grammar: src/ir.c:1-24;
 * reader rules: src/ir.c:458-554): `(model)`, `(param (data ...))`, quantized
 * params `(param NAME (f32 r c) (quant BITS AXIS (scale ...) (codes ...)))`
 * with codes one per element, range-checked and packed here exactly as the
 * reference packs them (src/ir.c:499-507: int8 as is, int4 two per byte,
 * element i in byte i/2, low nibble first, and `data` = code * scale in f32),
 * `(input)`, `(block)` with `const`, ops, `think` (src/ir.c:374-447) and
 * `scan` (src/ir.c:258-350), `(update)` (recorded: such models keep their rows
 * in order and are refused by the batch backend) and `(output)`.
 *
 * Atoms follow src/sexp.c:112-126: a token is a number when strtod consumes it
 * whole and it starts with a digit, or with + - . and is longer than one
 * character. Numbers are read with strtod and narrowed to float where the
 * reference narrows them (scales, data, constants, thresholds).
 *
 * The reader streams over the text: a 16.8 M-code int4 layer is packed as it
 * is read, without building an expression tree.
 *
 * Extension (not in the reference's grammar), for models whose weights are
 * too large to travel as text: a param's values may come from a file of raw
 * little-endian arrays, `(data-file PATH)` for f32 data, and inside `quant`
 * `(scale-file PATH)` (f32, one per channel) and `(codes-file PATH)` (int8,
 * one code per element, the text form's order), checked and packed exactly
 * like their text forms. PATH is one token (no blanks or parentheses). */
#include "tgm.h"

#include <ctype.h>
#include <limits.h>
#include <math.h>
#include <setjmp.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
	const char *s, *end;
	int line;
	jmp_buf fail;
	char *err;
	size_t errn;
	tgm_module *m;
	struct {
		char *name;
		int v;
	} *scope;
	int ns, scap;
	signed char *codes; /* codes read from a file, until packed */
	char **own;         /* strings the reader holds while a form is parsed (freed on failure too) */
	int nown, cown;
	int depth;          /* think and scan bodies open */
} Rd;

static void bad(Rd *r, const char *fmt, ...)
{
	va_list ap;
	int k = snprintf(r->err, r->errn, "tgir line %d: ", r->line);
	va_start(ap, fmt);
	if (k >= 0 && (size_t)k < r->errn) vsnprintf(r->err + k, r->errn - (size_t)k, fmt, ap);
	va_end(ap);
	longjmp(r->fail, 1);
}

static void *mem(Rd *r, size_t n, size_t sz)
{
	void *p = calloc(n ? n : 1, sz ? sz : 1);
	if (!p) bad(r, "out of memory");
	return p;
}

/* a copy of s, held by the reader until release_to(r, mark) with an earlier mark */
static char *own_str(Rd *r, const char *s)
{
	if (r->nown == r->cown) {
		const int cap = r->cown ? 2 * r->cown : 16;
		char **no = realloc(r->own, (size_t)cap * sizeof *no);
		if (!no) bad(r, "out of memory");
		r->own = no;
		r->cown = cap;
	}
	char *p = strdup(s);
	if (!p) bad(r, "out of memory");
	r->own[r->nown++] = p;
	return p;
}

static void release_to(Rd *r, int mark)
{
	while (r->nown > mark) free(r->own[--r->nown]);
}

/* skip blanks and ; comments, return the next character (0 at end) */
static int look(Rd *r)
{
	for (;;) {
		while (r->s < r->end && isspace((unsigned char)*r->s)) {
			if (*r->s == '\n') r->line++;
			r->s++;
		}
		if (r->s < r->end && *r->s == ';') {
			while (r->s < r->end && *r->s != '\n') r->s++;
			continue;
		}
		return r->s < r->end ? *r->s : 0;
	}
}

static void lp(Rd *r)
{
	if (look(r) != '(') bad(r, "expected '('");
	r->s++;
}

static void rp(Rd *r)
{
	if (look(r) != ')') bad(r, "expected ')'");
	r->s++;
}

typedef struct {
	char t[128];
	int num;
	double v;
} Atom;

static void atom(Rd *r, Atom *a)
{
	int c = look(r);
	if (!c || c == '(' || c == ')') bad(r, "expected a name or number");
	const char *b = r->s;
	while (r->s < r->end && !isspace((unsigned char)*r->s) && *r->s != '(' && *r->s != ')' && *r->s != ';' && *r->s != '"') r->s++;
	size_t n = (size_t)(r->s - b);
	if (n >= sizeof a->t) bad(r, "token too long");
	memcpy(a->t, b, n);
	a->t[n] = 0;
	char *e;
	a->v = strtod(a->t, &e);
	a->num = *e == 0 && (isdigit((unsigned char)a->t[0]) || ((a->t[0] == '-' || a->t[0] == '+' || a->t[0] == '.') && n > 1));
}

static double num(Rd *r, const char *what)
{
	Atom a;
	atom(r, &a);
	if (!a.num) bad(r, "expected a number for %s, got '%s'", what, a.t);
	return a.v;
}

static void sym(Rd *r, Atom *a)
{
	atom(r, a);
	if (a->num) bad(r, "expected a name, got '%s'", a->t);
}

static int sym_is(Rd *r, const char *want)
{
	Atom a;
	sym(r, &a);
	return strcmp(a.t, want) == 0;
}

/* the next form is a list whose head is the symbol `h` */
static int head_is(Rd *r, const char *h)
{
	if (look(r) != '(') return 0;
	const char *p = r->s + 1;
	while (p < r->end && isspace((unsigned char)*p)) p++;
	size_t n = strlen(h);
	return (size_t)(r->end - p) > n && !strncmp(p, h, n) && (isspace((unsigned char)p[n]) || p[n] == '(' || p[n] == ')');
}

long tgm_numel(const tgm_shape *s)
{
	long n = 1;
	for (int i = 0; i < s->rank; i++) n *= s->dim[i];
	return n;
}

static int same(const tgm_shape *a, const tgm_shape *b)
{
	if (a->rank != b->rank) return 0;
	for (int i = 0; i < a->rank; i++)
		if (a->dim[i] != b->dim[i]) return 0;
	return 1;
}

static tgm_shape type(Rd *r)
{
	tgm_shape s;
	memset(&s, 0, sizeof s);
	lp(r);
	if (!sym_is(r, "f32")) bad(r, "expected type (f32 d...)");
	while (look(r) != ')') {
		if (s.rank == TGM_MAXRANK) bad(r, "rank above %d", TGM_MAXRANK);
		double d = num(r, "a dimension");
		if (d < 1 || d != floor(d) || d > 2147483647.0) bad(r, "bad dimension");
		s.dim[s.rank++] = (int)d;
	}
	rp(r);
	return s;
}

static int value(Rd *r, int kind, const tgm_shape *sh, const char *name)
{
	tgm_module *m = r->m;
	if (m->nval == m->cap) {
		m->cap = m->cap ? 2 * m->cap : 64;
		tgm_value *nv = realloc(m->val, (size_t)m->cap * sizeof *nv);
		if (!nv) bad(r, "out of memory");
		m->val = nv;
	}
	tgm_value *v = &m->val[m->nval];
	memset(v, 0, sizeof *v);
	v->kind = kind;
	v->sh = *sh;
	v->n = tgm_numel(sh);
	if (name) {
		v->name = strdup(name);
		if (!v->name) bad(r, "out of memory");
	}
	return m->nval++;
}

static void bind(Rd *r, const char *name, int v)
{
	for (int i = 0; i < r->ns; i++)
		if (!strcmp(r->scope[i].name, name)) bad(r, "redefinition of '%s'", name);
	if (r->ns == r->scap) {
		r->scap = r->scap ? 2 * r->scap : 64;
		void *p = realloc(r->scope, (size_t)r->scap * sizeof *r->scope);
		if (!p) bad(r, "out of memory");
		r->scope = p;
	}
	r->scope[r->ns].name = strdup(name);
	r->scope[r->ns++].v = v;
}

static void unbind_to(Rd *r, int mark)
{
	while (r->ns > mark) free(r->scope[--r->ns].name);
}

static int ref(Rd *r)
{
	Atom a;
	sym(r, &a);
	for (int i = r->ns - 1; i >= 0; i--)
		if (!strcmp(r->scope[i].name, a.t)) return r->scope[i].v;
	bad(r, "undefined value '%s'", a.t);
	return -1;
}

static tgm_ins *emit(Rd *r, tgm_block *b)
{
	if (b->len == b->cap) {
		b->cap = b->cap ? 2 * b->cap : 8;
		tgm_ins *nv = realloc(b->v, (size_t)b->cap * sizeof *nv);
		if (!nv) bad(r, "out of memory");
		b->v = nv;
	}
	tgm_ins *in = &b->v[b->len++];
	memset(in, 0, sizeof *in);
	in->a[0] = in->a[1] = in->a[2] = -1;
	in->init = in->yield = in->halt = in->tid = in->stid = -1;
	return in;
}

static const struct {
	const char *name;
	int op, arity;
} OPS[] = {
	{ "add", TGM_ADD, 2 }, { "sub", TGM_SUB, 2 }, { "mul", TGM_MUL, 2 }, { "div", TGM_DIV, 2 }, { "max", TGM_MAX, 2 },
	{ "min", TGM_MIN, 2 }, { "neg", TGM_NEG, 1 }, { "tanh", TGM_TANH, 1 }, { "relu", TGM_RELU, 1 },
	{ "sigmoid", TGM_SIGMOID, 1 }, { "exp", TGM_EXP, 1 }, { "sqrt", TGM_SQRT, 1 }, { "gelu", TGM_GELU, 1 },
	{ "silu", TGM_SILU, 1 }, { "softplus", TGM_SOFTPLUS, 1 }, { "log", TGM_LOG, 1 }, { "sin", TGM_SIN, 1 },
	{ "cos", TGM_COS, 1 }, { "floor", TGM_FLOOR, 1 }, { "step", TGM_STEP, 1 }, { "matmul", TGM_MATMUL, 2 },
	{ "softmax", TGM_SOFTMAX, 1 }, { "rmsnorm", TGM_RMSNORM, 1 }, { "sum", TGM_SUM, 1 }, { "mean", TGM_MEAN, 1 },
	{ "transpose", TGM_TRANSPOSE, 1 }, { "outer", TGM_OUTER, 2 }, { "reshape", TGM_RESHAPE, 1 }, { "take", TGM_TAKE, 2 },
};

const char *tgm_op_name(int op)
{
	if (op == TGM_CONST) return "const";
	if (op == TGM_THINK) return "think";
	if (op == TGM_SCAN) return "scan";
	for (size_t i = 0; i < sizeof OPS / sizeof OPS[0]; i++)
		if (OPS[i].op == op) return OPS[i].name;
	return "?";
}

static void items(Rd *r, tgm_block *b, int in_think);

static int *ints(Rd *r, int n) { return mem(r, (size_t)(n ? n : 1), sizeof(int)); }

static void scan_form(Rd *r, tgm_block *b)
{
	tgm_module *m = r->m;
	double T = num(r, "scan steps");
	if (T < 1 || T != floor(T) || T > INT_MAX) bad(r, "malformed scan (steps)");
	Atom a;
	sym(r, &a);
	if (strcmp(a.t, "forward") && strcmp(a.t, "reverse")) bad(r, "malformed scan (direction)");
	int rev = !strcmp(a.t, "reverse"), stid = -1;
	if (look(r) != '(') {
		sym(r, &a);
		if (strcmp(a.t, "steps")) bad(r, "malformed scan");
		stid = m->nthink++;
	}
	enum { MX = 32 };
	const int held = r->nown;
	char *cname[MX], *xname[MX], *yname[MX];
	int c[MX], ci[MX], cn[MX], x[MX], xt[MX], yv[MX], nc = 0, nx = 0, ny = 0;
	tgm_shape ysh[MX];
	while (head_is(r, "carry")) {
		if (nc == MX) bad(r, "too many carries");
		lp(r);
		sym(r, &a);
		sym(r, &a);
		cname[nc] = own_str(r, a.t);
		tgm_shape sh = type(r);
		ci[nc] = ref(r);
		rp(r);
		if (!same(&sh, &m->val[ci[nc]].sh)) bad(r, "carry type differs from its initial value");
		c[nc] = value(r, TGM_TMP, &sh, NULL);
		nc++;
	}
	if (!nc) bad(r, "malformed scan (needs a carry)");
	while (head_is(r, "in")) {
		if (nx == MX) bad(r, "too many sequences");
		lp(r);
		sym(r, &a);
		sym(r, &a);
		xname[nx] = own_str(r, a.t);
		tgm_shape sh = type(r);
		x[nx] = ref(r);
		rp(r);
		tgm_shape row = m->val[x[nx]].sh;
		if (row.rank < 1 || row.dim[0] != (int)T) bad(r, "sequence does not have %d steps along its first axis", (int)T);
		for (int d = 1; d < row.rank; d++) row.dim[d - 1] = row.dim[d];
		row.rank--;
		if (!same(&sh, &row)) bad(r, "slice type differs from a row of its sequence");
		xt[nx] = value(r, TGM_TMP, &sh, NULL);
		nx++;
	}
	int mark = r->ns;
	for (int k = 0; k < nc; k++) bind(r, cname[k], c[k]);
	for (int j = 0; j < nx; j++) bind(r, xname[j], xt[j]);
	if (!head_is(r, "body")) bad(r, "malformed scan (body)");
	int at = b->len;
	emit(r, b);
	tgm_block *body = mem(r, 1, sizeof *body);
	b->v[at].body = body; /* owned by the instruction from here on, so a failure below frees it */
	lp(r);
	sym(r, &a);
	items(r, body, 0);
	rp(r);
	for (int k = 0; k < nc; k++) {
		if (!head_is(r, "next")) bad(r, "malformed scan (next)");
		lp(r);
		sym(r, &a);
		if (ref(r) != c[k]) bad(r, "'next' entries must follow the carries in order");
		cn[k] = ref(r);
		rp(r);
		if (!same(&m->val[cn[k]].sh, &m->val[c[k]].sh)) bad(r, "next value shape differs from its carry");
	}
	while (look(r) == '(') {
		if (!head_is(r, "emit") || ny == MX) bad(r, "malformed scan (emit)");
		lp(r);
		sym(r, &a);
		sym(r, &a);
		yname[ny] = own_str(r, a.t);
		ysh[ny] = type(r);
		yv[ny] = ref(r);
		rp(r);
		tgm_shape want = m->val[yv[ny]].sh;
		if (want.rank == TGM_MAXRANK) bad(r, "stack rank above %d", TGM_MAXRANK);
		for (int d = want.rank; d > 0; d--) want.dim[d] = want.dim[d - 1];
		want.dim[0] = (int)T;
		want.rank++;
		if (!same(&ysh[ny], &want)) bad(r, "emit type differs from the stack of its value");
		ny++;
	}
	unbind_to(r, mark);
	for (int k = 0; k < nc; k++) bind(r, cname[k], c[k]);
	tgm_ins *in = &b->v[at];
	in->op = TGM_SCAN;
	in->T = (int)T;
	in->reverse = rev;
	in->stid = stid;
	in->nc = nc;
	in->nx = nx;
	in->ny = ny;
	in->c = ints(r, nc);
	in->cinit = ints(r, nc);
	in->cnext = ints(r, nc);
	in->x = ints(r, nx);
	in->xt = ints(r, nx);
	in->y = ints(r, ny);
	in->ys = ints(r, ny);
	for (int k = 0; k < nc; k++) {
		in->c[k] = c[k];
		in->cinit[k] = ci[k];
		in->cnext[k] = cn[k];
	}
	for (int j = 0; j < nx; j++) {
		in->x[j] = x[j];
		in->xt[j] = xt[j];
	}
	for (int y = 0; y < ny; y++) {
		in->y[y] = yv[y];
		in->ys[y] = value(r, TGM_TMP, &ysh[y], NULL);
		bind(r, yname[y], in->ys[y]);
	}
	release_to(r, held);
	in = &b->v[at];
	in->out = c[0];
}

/* bodies nest at most this deep (the parser recurses once per level) */
#define TGM_MAX_DEPTH 64

static void block_items(Rd *r, tgm_block *b, int in_think);

static void items(Rd *r, tgm_block *b, int in_think)
{
	if (++r->depth > TGM_MAX_DEPTH) bad(r, "think and scan bodies nested more than %d deep", TGM_MAX_DEPTH);
	block_items(r, b, in_think);
	r->depth--;
}

static void block_items(Rd *r, tgm_block *b, int in_think)
{
	tgm_module *m = r->m;
	Atom a, nm;
	for (;;) {
		if (look(r) == ')' || (in_think && head_is(r, "yield"))) return;
		if (head_is(r, "scan")) {
			lp(r);
			sym(r, &a);
			scan_form(r, b);
			rp(r);
			continue;
		}
		lp(r);
		sym(r, &nm);
		tgm_shape decl = type(r);
		lp(r);
		sym(r, &a);
		int out;
		if (!strcmp(a.t, "const")) {
			double k = num(r, "const");
			rp(r);
			out = value(r, TGM_TMP, &decl, NULL);
			tgm_ins *in = emit(r, b);
			in->op = TGM_CONST;
			in->k = (float)k;
			in->out = out;
		} else if (!strcmp(a.t, "think")) {
			int init = ref(r);
			double budget = num(r, "think budget");
			/* (above INT_MAX the reference's int conversion is undefined: refused here) */
			if (!(budget >= 1 && budget <= INT_MAX)) bad(r, "malformed think budget");
			Atom e;
			atom(r, &e);
			double eps = -1;
			if (e.num) {
				if (e.v < 0) bad(r, "malformed think threshold");
				eps = e.v;
			} else if (strcmp(e.t, "none")) {
				bad(r, "malformed think threshold");
			}
			if (!same(&decl, &m->val[init].sh)) bad(r, "declared %s type differs from the think state", nm.t);
			out = value(r, TGM_TMP, &decl, NULL);
			int at = b->len;
			emit(r, b);
			int tid = m->nthink++;
			tgm_block *body = mem(r, 1, sizeof *body);
			b->v[at].body = body; /* owned by the instruction from here on */
			int mark = r->ns;
			bind(r, nm.t, out);
			items(r, body, 1);
			if (!head_is(r, "yield")) bad(r, "think (missing yield)");
			lp(r);
			sym(r, &a);
			int y = ref(r);
			rp(r);
			int halt = -1;
			double thr = 0;
			if (head_is(r, "halt")) {
				lp(r);
				sym(r, &a);
				halt = ref(r);
				thr = num(r, "halt threshold");
				rp(r);
				if (!(thr > 0 && thr < 1) || eps >= 0) bad(r, "think halt (value, threshold in (0, 1); no until)");
				if (m->val[halt].sh.rank != 0) bad(r, "halting value must be a scalar");
			}
			rp(r);
			if (!same(&m->val[y].sh, &decl)) bad(r, "yield shape differs from state shape");
			unbind_to(r, mark);
			tgm_ins *in = &b->v[at];
			in->op = TGM_THINK;
			in->out = out;
			in->init = init;
			in->maxit = (int)budget;
			in->eps = eps < 0 ? -1.0f : (float)eps;
			in->tid = tid;
			in->body = body;
			in->yield = y;
			in->halt = halt;
			in->hthr = (float)thr;
		} else {
			int op = -1, ar = 0, na = 0, args[3];
			for (size_t i = 0; i < sizeof OPS / sizeof OPS[0]; i++)
				if (!strcmp(OPS[i].name, a.t)) {
					op = OPS[i].op;
					ar = OPS[i].arity;
				}
			if (op < 0) bad(r, "op '%s' is not supported by the batch backend", a.t);
			while (look(r) != ')') {
				if (na == 3) bad(r, "too many operands");
				args[na++] = ref(r);
			}
			rp(r);
			if (na != ar) bad(r, "'%s' takes %d operand(s), got %d", a.t, ar, na);
			if (op == TGM_RESHAPE && m->val[args[0]].n != tgm_numel(&decl)) bad(r, "reshape changes the element count");
			out = value(r, TGM_TMP, &decl, NULL);
			tgm_ins *in = emit(r, b);
			in->op = op;
			in->out = out;
			in->na = na;
			for (int j = 0; j < na; j++) in->a[j] = args[j];
		}
		rp(r);
		bind(r, nm.t, out);
	}
}

/* `bytes` of raw data from the file named by the next token into dst */
static void file_data(Rd *r, void *dst, size_t bytes, const char *what)
{
	Atom path;
	atom(r, &path);
	FILE *f = fopen(path.t, "rb");
	if (!f) bad(r, "cannot open %s file '%s'", what, path.t);
	const size_t got = fread(dst, 1, bytes, f);
	const int extra = fgetc(f) != EOF;
	fclose(f);
	if (got != bytes || extra) bad(r, "%s file '%s' must hold exactly %zu bytes", what, path.t, bytes);
}

static void param_form(Rd *r, int kind)
{
	tgm_module *m = r->m;
	Atom nm, a;
	sym(r, &nm);
	tgm_shape sh = type(r);
	int v = value(r, kind, &sh, nm.t);
	tgm_value *x = &m->val[v];
	lp(r);
	sym(r, &a);
	if (!strcmp(a.t, "quant") && kind == TGM_PARAM) {
		double bits = num(r, "quant bits"), axis = num(r, "quant axis");
		if (bits != 8 && bits != 4) bad(r, "malformed quant bits (8 or 4)");
		if ((axis != 0 && axis != 1) || sh.rank != 2) bad(r, "malformed quant axis (0 or 1, rank-2 param)");
		x->qbits = (int)bits;
		x->qaxis = (int)axis;
		long nch = sh.dim[x->qaxis];
		x->qs = mem(r, (size_t)nch, sizeof(float));
		x->q = mem(r, (size_t)(x->qbits == 8 ? x->n : (x->n + 1) / 2), 1);
		x->data = mem(r, (size_t)x->n, sizeof(float));
		lp(r);
		Atom h;
		sym(r, &h);
		if (!strcmp(h.t, "scale-file")) {
			file_data(r, x->qs, (size_t)nch * sizeof(float), "scale");
		} else {
			if (strcmp(h.t, "scale")) bad(r, "malformed quant scales");
			for (long j = 0; j < nch; j++) {
				if (look(r) == ')') bad(r, "quant needs one scale per channel");
				x->qs[j] = (float)num(r, "a scale");
			}
		}
		rp(r);
		lp(r);
		sym(r, &h);
		signed char *raw = NULL; /* codes from a file (owned by r until freed, so a failure frees them) */
		if (!strcmp(h.t, "codes-file")) {
			raw = r->codes = mem(r, (size_t)x->n, 1);
			file_data(r, raw, (size_t)x->n, "codes");
		} else if (strcmp(h.t, "codes")) {
			bad(r, "malformed quant codes");
		}
		int lim = x->qbits == 8 ? 127 : 7;
		for (long j = 0; j < x->n; j++) {
			double cd;
			if (raw) {
				cd = raw[j];
			} else {
				if (look(r) == ')') bad(r, "quant needs one code per element");
				cd = num(r, "a code");
			}
			if (cd != floor(cd) || fabs(cd) > lim) bad(r, "code out of range");
			int code = (int)cd;
			if (x->qbits == 8) x->q[j] = (unsigned char)(signed char)code;
			else if (j & 1) x->q[j >> 1] = (unsigned char)((x->q[j >> 1] & 0x0f) | ((unsigned)code << 4));
			else x->q[j >> 1] = (unsigned char)((x->q[j >> 1] & 0xf0) | (code & 0x0f));
			long ch = x->qaxis == 0 ? j / sh.dim[1] : j % sh.dim[1];
			x->data[j] = (float)code * x->qs[ch];
		}
		free(raw);
		r->codes = NULL;
		rp(r);
		rp(r);
	} else if (!strcmp(a.t, "data-file")) {
		x->data = mem(r, (size_t)x->n, sizeof(float));
		file_data(r, x->data, (size_t)x->n * sizeof(float), "data");
		rp(r);
	} else if (!strcmp(a.t, "data")) {
		x->data = mem(r, (size_t)x->n, sizeof(float));
		long j = 0;
		while (look(r) != ')') {
			double d = num(r, "data");
			if (j < x->n) x->data[j] = (float)d;
			j++;
		}
		if (j != x->n) bad(r, "param '%s' needs %ld values, has %ld", nm.t, x->n, j);
		rp(r);
	} else {
		bad(r, "malformed %s", kind == TGM_STATE ? "state" : "param");
	}
	rp(r);
	bind(r, nm.t, v);
}

tgm_module *tgm_read(const char *text, size_t len, char *err, size_t errn)
{
	Rd r;
	memset(&r, 0, sizeof r);
	r.s = text;
	r.end = text + len;
	r.line = 1;
	r.err = err;
	r.errn = errn;
	r.m = calloc(1, sizeof *r.m);
	if (!r.m) {
		snprintf(err, errn, "out of memory");
		return NULL;
	}
	r.m->output = -1;
	if (setjmp(r.fail)) {
		unbind_to(&r, 0);
		free(r.scope);
		free(r.codes);
		release_to(&r, 0);
		free(r.own);
		tgm_free(r.m);
		return NULL;
	}
	Atom a;
	int seen_block = 0, seen_out = 0;
	lp(&r);
	if (!sym_is(&r, "tgir")) bad(&r, "expected (tgir 1 ...)");
	if (num(&r, "version") != 1) bad(&r, "unsupported TGIR version");
	while (look(&r) != ')') {
		lp(&r);
		sym(&r, &a);
		if (!strcmp(a.t, "model")) {
			if (r.m->name) bad(&r, "malformed model");
			sym(&r, &a);
			r.m->name = strdup(a.t);
			rp(&r);
			continue;
		}
		if (!r.m->name) bad(&r, "(model ...) must come first");
		if (!strcmp(a.t, "param") || !strcmp(a.t, "state")) {
			if (seen_block) bad(&r, "params come before the block");
			param_form(&r, strcmp(a.t, "state") ? TGM_PARAM : TGM_STATE);
		} else if (!strcmp(a.t, "input")) {
			if (seen_block) bad(&r, "inputs come before the block");
			Atom nm;
			sym(&r, &nm);
			tgm_shape sh = type(&r);
			rp(&r);
			int v = value(&r, TGM_INPUT, &sh, nm.t);
			r.m->val[v].index = r.m->ninputs;
			r.m->val[v].in_off = r.m->per;
			r.m->per += r.m->val[v].n;
			int *ni = realloc(r.m->inputs, (size_t)(r.m->ninputs + 1) * sizeof *ni);
			if (!ni) bad(&r, "out of memory");
			r.m->inputs = ni;
			r.m->inputs[r.m->ninputs++] = v;
			bind(&r, nm.t, v);
		} else if (!strcmp(a.t, "block")) {
			if (seen_block) bad(&r, "duplicate block");
			seen_block = 1;
			items(&r, &r.m->top, 0);
			rp(&r);
		} else if (!strcmp(a.t, "update")) {
			if (!seen_block) bad(&r, "malformed update");
			for (int depth = 1; depth;) { /* recorded only: the backend refuses stateful models */
				int c = look(&r);
				if (!c) bad(&r, "unterminated update");
				depth += c == '(' ? 1 : c == ')' ? -1 : 0;
				r.s++;
			}
			r.m->nupd++;
		} else if (!strcmp(a.t, "output")) {
			if (!seen_block || seen_out) bad(&r, "malformed output");
			seen_out = 1;
			r.m->output = ref(&r);
			rp(&r);
		} else {
			bad(&r, "unknown top-level form '%s'", a.t);
		}
	}
	rp(&r);
	if (look(&r)) bad(&r, "text after the (tgir ...) form");
	if (!r.m->ninputs) bad(&r, "module has no inputs");
	if (!seen_out) bad(&r, "missing (output ...)");
	r.m->nout = r.m->val[r.m->output].n;
	unbind_to(&r, 0);
	free(r.scope);
	free(r.own);
	return r.m;
}

static void free_block(tgm_block *b)
{
	for (int i = 0; i < b->len; i++) {
		tgm_ins *in = &b->v[i];
		if (in->body) {
			free_block(in->body);
			free(in->body);
		}
		if (in->op == TGM_SCAN) {
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

void tgm_free(tgm_module *m)
{
	if (!m) return;
	for (int i = 0; i < m->nval; i++) {
		free(m->val[i].name);
		free(m->val[i].data);
		free(m->val[i].q);
		free(m->val[i].qs);
	}
	free(m->val);
	free(m->inputs);
	free_block(&m->top);
	free(m->name);
	free(m);
}

int tgm_code(const tgm_value *v, long i)
{
	if (v->qbits == 8) return (signed char)v->q[i];
	int b = (signed char)v->q[i >> 1];
	return (i & 1) ? (b >> 4) : (int)(signed char)(unsigned char)((unsigned)b << 4) >> 4;
}
