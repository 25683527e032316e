/* The surface-language front end (tg_front.h): .tg source -> canonical TGIR.
 *
 * Pipeline, each stage restating the reference's behaviour for the subset of
 * the language the batch backend runs:
 *   files     the root file and its imports (src/lower.c:686-760): an import
 *             is resolved against the importing file's directory and merged
 *             once; an imported file contributes its params, states and defs
 *             other than `forward`;
 *   tokens    indentation blocks, brackets that suspend line ends, `#`
 *             comments, strtod numbers (src/parse.c:56-132);
 *   syntax    declarations, statements and expressions with the reference's
 *             precedence and negative-literal folding (src/parse.c:134-542);
 *   lowering  params materialised (zeros, ones, fill, rand, file, env,
 *             literals), every def inlined at its call, names renamed into SSA
 *             values, think and scan loops with their scoping rules, `dot`,
 *             `mse`/`bce`/`xent`, `rope`, `attention`, `take_along` and
 *             `reshape` expanded into table operations (src/lower.c:81-650);
 *   liveness  instructions unreachable from the output and the state updates
 *             removed, scan carries and stacks pruned (src/lower.c:823-905);
 *   text      the canonical writer: params and states in declaration order,
 *             inputs, then the block with temporaries numbered in the order a
 *             reader recreates them (src/ir.c:40-202).
 * Operations the batch backend does not run (autodiff, training, sparse and
 * memory ops, topk, suffix matching) are refused with a message. Errors carry
 * the reference's diagnostic text as "file:line: message". */
#define _GNU_SOURCE
#include "tg_front.h"

#include <ctype.h>
#include <math.h>
#include <setjmp.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define MAXRANK 4

/* ------------------------------------------------------------ context --- */

typedef struct {
	int rank, dim[MAXRANK];
} Sh;

enum { K_TMP, K_PARAM, K_STATE, K_INPUT };

typedef struct {
	int kind, dead;
	Sh sh;
	const char *name; /* NULL for temporaries */
	float *data;      /* params and states */
} Val;

typedef struct Blk Blk;

typedef struct {
	int op, out, na, a[3];
	float k;                    /* const */
	int init, maxit, yield, halt; /* think */
	float eps, hthr;
	Blk *body;                  /* think and scan */
	int T, nc, nx, ny;          /* scan */
	int *c, *cinit, *cnext, *x, *xt, *y, *ys;
} Ins;

struct Blk {
	Ins *v;
	int len, cap;
};

typedef struct {
	char **p;
	int n, cap;
} Mem;

typedef struct {
	jmp_buf jb;
	char *err;
	size_t errn;
	Mem mem;
	/* module */
	const char *name;
	Val *val;
	int nval, capval;
	int *inputs, ninputs;
	int output;
	int *ust, *usrc, *urows, nupd;
	Blk top;
} F;

static void *fa(F *f, size_t n)
{
	void *p = calloc(1, n ? n : 1);
	if (!p || (f->mem.n == f->mem.cap && !(f->mem.p = realloc(f->mem.p, (size_t)(f->mem.cap = f->mem.cap ? 2 * f->mem.cap : 256) * sizeof *f->mem.p)))) {
		free(p);
		snprintf(f->err, f->errn, "out of memory");
		longjmp(f->jb, 1);
	}
	f->mem.p[f->mem.n++] = p;
	return p;
}

static void *fgrow(F *f, void *old, size_t n) /* a larger copy (the old block stays owned until the end) */
{
	void *p = fa(f, n);
	(void)old;
	return p;
}

static char *fstr(F *f, const char *s, size_t n)
{
	char *d = fa(f, n + 1);
	memcpy(d, s, n);
	return d;
}

static void fail(F *f, const char *file, int line, const char *fmt, ...)
{
	char msg[512];
	va_list ap;
	va_start(ap, fmt);
	vsnprintf(msg, sizeof msg, fmt, ap);
	va_end(ap);
	if (file) snprintf(f->err, f->errn, "%s:%d: %s", file, line, msg);
	else snprintf(f->err, f->errn, "%s", msg);
	longjmp(f->jb, 1);
}

/* ------------------------------------------------------------- shapes --- */

static int numel(const Sh *s)
{
	int n = 1;
	for (int i = 0; i < s->rank; i++) n *= s->dim[i];
	return n;
}

static int sheq(const Sh *a, const Sh *b)
{
	if (a->rank != b->rank) return 0;
	for (int i = 0; i < a->rank; i++)
		if (a->dim[i] != b->dim[i]) return 0;
	return 1;
}

static const char *shstr(const Sh *s, char *buf) /* "(f32 d...)"; buf holds 64 bytes */
{
	int o = snprintf(buf, 64, "(f32");
	for (int i = 0; i < s->rank && o < 64; i++) o += snprintf(buf + o, (size_t)(64 - o), " %d", s->dim[i]);
	if (o < 64) snprintf(buf + o, (size_t)(64 - o), ")");
	return buf;
}

static int broadcast(const Sh *a, const Sh *b, Sh *o)
{
	Sh r = { 0, { 0 } };
	r.rank = a->rank > b->rank ? a->rank : b->rank;
	for (int i = 1; i <= r.rank; i++) {
		int x = i <= a->rank ? a->dim[a->rank - i] : 1, y = i <= b->rank ? b->dim[b->rank - i] : 1;
		if (x != y && x != 1 && y != 1) return 0;
		r.dim[r.rank - i] = x == 1 ? y : x;
	}
	*o = r;
	return 1;
}

/* ---------------------------------------------------------- op table --- */

enum { C_CONST, C_BIN, C_UN, C_MATMUL, C_ROW, C_RED, C_TRANS, C_OUTER, C_TAKE, C_RESHAPE, C_THINK, C_SCAN, C_OTHER };

typedef struct {
	const char *name;
	int arity, cls;
} Op;

/* The reference's operation names (src/ops.c:7-51); C_OTHER ones exist in
 * the language but not in the batch backend. */
static const Op OPS[] = {
	{ "const", 0, C_CONST },     { "add", 2, C_BIN },       { "sub", 2, C_BIN },       { "mul", 2, C_BIN },
	{ "div", 2, C_BIN },         { "max", 2, C_BIN },       { "min", 2, C_BIN },       { "neg", 1, C_UN },
	{ "tanh", 1, C_UN },         { "relu", 1, C_UN },       { "sigmoid", 1, C_UN },    { "exp", 1, C_UN },
	{ "sqrt", 1, C_UN },         { "gelu", 1, C_UN },       { "silu", 1, C_UN },       { "softplus", 1, C_UN },
	{ "log", 1, C_UN },          { "matmul", 2, C_MATMUL }, { "softmax", 1, C_ROW },   { "rmsnorm", 1, C_ROW },
	{ "sum", 1, C_RED },         { "mean", 1, C_RED },      { "transpose", 1, C_TRANS }, { "outer", 2, C_OUTER },
	{ "step", 1, C_UN },         { "spmm", 2, C_OTHER },    { "spmm_t", 3, C_OTHER },  { "spmm_dx", 3, C_OTHER },
	{ "active", 2, C_OTHER },    { "take", 2, C_TAKE },     { "take_t", 3, C_OTHER },  { "spmm_tc", 3, C_OTHER },
	{ "sin", 1, C_UN },          { "cos", 1, C_UN },        { "reshape", 1, C_RESHAPE }, { "floor", 1, C_UN },
	{ "sum_to", 2, C_OTHER },    { "topk", 1, C_OTHER },    { "memscan", 3, C_OTHER }, { "memscan_t", 3, C_OTHER },
	{ "sufmatch", 1, C_OTHER },  { "think", 0, C_THINK },   { "scan", 0, C_SCAN },
};
#define NOPS ((int)(sizeof OPS / sizeof *OPS))

static int op_of(const char *name)
{
	for (int i = 0; i < NOPS; i++)
		if (OPS[i].cls != C_CONST && OPS[i].cls != C_THINK && OPS[i].cls != C_SCAN && !strcmp(OPS[i].name, name)) return i;
	return -1;
}

static int op_id(const char *name) /* an op this file emits by name */
{
	for (int i = 0; i < NOPS; i++)
		if (!strcmp(OPS[i].name, name)) return i;
	return -1;
}

/* shape inference (src/ops.c:97-330, the classes above); NULL on success */
static const char *infer(int op, const Sh *a, int na, Sh *o, char *err)
{
	char s0[64], s1[64];
	const Op *oi = &OPS[op];
	if (na != oi->arity) return snprintf(err, 300, "'%s' takes %d operand(s), got %d", oi->name, oi->arity, na), err;
	memset(o, 0, sizeof *o);
	switch (oi->cls) {
	case C_BIN:
		if (broadcast(&a[0], &a[1], o)) return NULL;
		snprintf(err, 300, "'%s' shape mismatch %s vs %s (dimensions are compared from the right; each pair must be equal or one of them 1)",
			 oi->name, shstr(&a[0], s0), shstr(&a[1], s1));
		return err;
	case C_UN: *o = a[0]; return NULL;
	case C_MATMUL: {
		int ra = a[0].rank, rb = a[1].rank, ka = ra >= 1 ? a[0].dim[ra - 1] : -1, kb = rb == 3 ? a[1].dim[1] : rb >= 1 ? a[1].dim[0] : -1;
		if (ra < 1 || ra > 3 || rb < 1 || rb > 3 || ka != kb || (rb == 3 && (ra != 3 || a[0].dim[0] != a[1].dim[0]))) {
			snprintf(err, 300, "'matmul' incompatible operands %s @ %s", shstr(&a[0], s0), shstr(&a[1], s1));
			return err;
		}
		for (int i = 0; i < ra - 1; i++) o->dim[o->rank++] = a[0].dim[i];
		if (rb >= 2) o->dim[o->rank++] = a[1].dim[rb - 1];
		return NULL;
	}
	case C_ROW:
		if (a[0].rank == 0) return snprintf(err, 300, "'%s' needs rank >= 1", oi->name), err;
		*o = a[0];
		return NULL;
	case C_RED: return NULL;
	case C_TRANS:
		if (a[0].rank != 2 && a[0].rank != 3) return snprintf(err, 300, "'transpose' needs rank 2, or rank 3 (the last two axes swap)"), err;
		*o = a[0];
		o->dim[o->rank - 2] = a[0].dim[a[0].rank - 1];
		o->dim[o->rank - 1] = a[0].dim[a[0].rank - 2];
		return NULL;
	case C_OUTER:
		if (a[0].rank != 1 || a[1].rank != 1) {
			snprintf(err, 300, "'outer' needs two vectors, got %s and %s", shstr(&a[0], s0), shstr(&a[1], s1));
			return err;
		}
		o->rank = 2;
		o->dim[0] = a[0].dim[0];
		o->dim[1] = a[1].dim[0];
		return NULL;
	case C_TAKE:
		if (a[0].rank < 1 || a[1].rank != 1) {
			snprintf(err, 300, "'take' needs a tensor (D, ...) and row indices (n), got %s and %s", shstr(&a[0], s0), shstr(&a[1], s1));
			return err;
		}
		*o = a[0];
		o->dim[0] = a[1].dim[0];
		return NULL;
	case C_RESHAPE:
		return snprintf(err, 300, "'reshape' takes a tensor and its new dimensions, e.g. reshape(x, 4, 8)"), err;
	default: break;
	}
	return snprintf(err, 300, "'%s' is not a value operation", oi->name), err;
}

/* ------------------------------------------------------------- module --- */

static int newval(F *f, int kind, const Sh *sh, const char *name)
{
	if (f->nval == f->capval) {
		int cap = f->capval ? 2 * f->capval : 64;
		Val *v = fgrow(f, f->val, (size_t)cap * sizeof *v);
		if (f->nval) memcpy(v, f->val, (size_t)f->nval * sizeof *v);
		f->val = v;
		f->capval = cap;
	}
	Val *v = &f->val[f->nval];
	memset(v, 0, sizeof *v);
	v->kind = kind;
	v->sh = *sh;
	v->name = name;
	if (kind == K_INPUT) {
		int *in = fa(f, (size_t)(f->ninputs + 1) * sizeof *in);
		if (f->ninputs) memcpy(in, f->inputs, (size_t)f->ninputs * sizeof *in);
		in[f->ninputs++] = f->nval;
		f->inputs = in;
	}
	return f->nval++;
}

static int push(F *f, Blk *b) /* index of a new zeroed instruction */
{
	if (b->len == b->cap) {
		int cap = b->cap ? 2 * b->cap : 16;
		Ins *v = fgrow(f, b->v, (size_t)cap * sizeof *v);
		if (b->len) memcpy(v, b->v, (size_t)b->len * sizeof *v);
		b->v = v;
		b->cap = cap;
	}
	memset(&b->v[b->len], 0, sizeof *b->v);
	b->v[b->len].halt = -1;
	return b->len++;
}

static int *ints_add(F *f, int *a, int n, int x)
{
	int *r = fa(f, (size_t)(n + 1) * sizeof *r);
	if (n) memcpy(r, a, (size_t)n * sizeof *r);
	r[n] = x;
	return r;
}

/* ---------------------------------------------------------- tokens --- */

enum { T_NAME, T_NUM, T_STR, T_OP, T_NL, T_INDENT, T_DEDENT, T_EOF };

typedef struct {
	int k, line;
	const char *s;
	double n;
} Tok;

typedef struct {
	F *f;
	const char *file;
	Tok *t;
	int n, cap, i;
} P;

static void tok(P *p, int k, const char *s, size_t len, double n, int line)
{
	if (p->n == p->cap) {
		int cap = p->cap ? 2 * p->cap : 256;
		Tok *t = fgrow(p->f, p->t, (size_t)cap * sizeof *t);
		if (p->n) memcpy(t, p->t, (size_t)p->n * sizeof *t);
		p->t = t;
		p->cap = cap;
	}
	p->t[p->n++] = (Tok){ k, line, fstr(p->f, s, len), n };
}

static void lex(P *p, const char *src)
{
	int col_stack[64], sp = 0, line = 1, depth = 0, bol = 1;
	col_stack[0] = 0;
	const char *c = src;
	while (*c) {
		if (bol && depth == 0) { /* a line's indentation */
			int col = 0;
			while (*c == ' ') col++, c++;
			if (*c == '\t') fail(p->f, p->file, line, "tabs are not allowed for indentation");
			if (*c == '\n' || *c == '#' || *c == '\r' || !*c) { /* blank or comment-only line */
				while (*c && *c != '\n') c++;
				if (*c) c++, line++;
				continue;
			}
			bol = 0;
			if (col > col_stack[sp]) {
				if (sp == 63) fail(p->f, p->file, line, "nesting too deep");
				col_stack[++sp] = col;
				tok(p, T_INDENT, "", 0, 0, line);
			} else {
				while (col < col_stack[sp]) sp--, tok(p, T_DEDENT, "", 0, 0, line);
				if (col != col_stack[sp]) fail(p->f, p->file, line, "inconsistent dedent");
			}
		}
		if (*c == '\n') {
			if (depth == 0) tok(p, T_NL, "", 0, 0, line), bol = 1;
			c++, line++;
		} else if (*c == ' ' || *c == '\r' || *c == '\t') {
			c++;
		} else if (*c == '#') {
			while (*c && *c != '\n') c++;
		} else if (isalpha((unsigned char)*c) || *c == '_') {
			const char *s = c;
			while (isalnum((unsigned char)*c) || *c == '_') c++;
			tok(p, T_NAME, s, (size_t)(c - s), 0, line);
		} else if (isdigit((unsigned char)*c) || (*c == '.' && isdigit((unsigned char)c[1]))) {
			char *e;
			double v = strtod(c, &e);
			tok(p, T_NUM, c, (size_t)(e - c), v, line);
			c = e;
		} else if (*c == '"') {
			const char *s = ++c;
			while (*c && *c != '"' && *c != '\n') c++;
			if (*c != '"') fail(p->f, p->file, line, "unterminated string");
			tok(p, T_STR, s, (size_t)(c - s), 0, line);
			c++;
		} else if (c[0] == '-' && c[1] == '>') {
			tok(p, T_OP, c, 2, 0, line);
			c += 2;
		} else if (strchr("+-*/@()[],:=", *c)) {
			if (*c == '(' || *c == '[') depth++;
			if ((*c == ')' || *c == ']') && depth > 0) depth--;
			tok(p, T_OP, c, 1, 0, line);
			c++;
		} else {
			fail(p->f, p->file, line, "unexpected character '%c'", *c);
		}
	}
	if (p->n && p->t[p->n - 1].k != T_NL) tok(p, T_NL, "", 0, 0, line);
	while (sp > 0) sp--, tok(p, T_DEDENT, "", 0, 0, line);
	tok(p, T_EOF, "", 0, 0, line);
}

/* ------------------------------------------------------------ syntax --- */

enum { E_NUM, E_REF, E_CALL };

typedef struct Ex {
	int kind, line, nargs;
	double num;
	const char *name;
	struct Ex **args;
} Ex;

enum { S_SET, S_RETURN, S_THINK, S_SCAN, S_EMIT, S_UPDATE, S_TRAIN };

typedef struct St {
	int kind, line;
	const char *name;
	Ex *e, *rows;
	/* think */
	int maxit, has_halt;
	double eps, hthr;
	const char *halt;
	/* scan */
	const char **cs, **xn;
	Ex **xe;
	int ncs, nx;
	struct St **body;
	int nbody, bline; /* bline: the body's first line */
} St;

enum { I_ZEROS, I_ONES, I_FILL, I_RAND, I_FILE, I_ENV, I_DATA };

typedef struct {
	int kind, nv, line, cap;
	double *v;
	const char *str;
} Init;

enum { D_MODEL, D_PARAM, D_STATE, D_DEF, D_IMPORT };

typedef struct {
	int kind, line, nargs;
	const char *name, *str;
	Sh sh;
	Init init;
	const char **an;
	Sh *as;
	St **body;
	int nbody, bline;
} Decl;

static const char *KW[] = { "model", "param", "def", "return", "think", "for", "until", "f32", "import", "state", "update", "train", "with", "over", "scan", "emit", NULL };

static Tok *peek(P *p) { return &p->t[p->i]; }
static Tok *next(P *p)
{
	Tok *t = &p->t[p->i];
	if (t->k != T_EOF) p->i++;
	return t;
}

static const char *desc(Tok *t)
{
	switch (t->k) {
	case T_NL: return "end of line";
	case T_INDENT: return "indent";
	case T_DEDENT: return "dedent";
	case T_EOF: return "end of file";
	default: return t->s;
	}
}

static int isop(Tok *t, const char *s) { return t->k == T_OP && !strcmp(t->s, s); }
static int iskw(Tok *t, const char *s) { return t->k == T_NAME && !strcmp(t->s, s); }

static void want_op(P *p, const char *s)
{
	Tok *t = next(p);
	if (!isop(t, s)) fail(p->f, p->file, t->line, "expected '%s', got '%s'", s, desc(t));
}

static Tok *want(P *p, int k, const char *what)
{
	Tok *t = next(p);
	if (t->k != k) fail(p->f, p->file, t->line, "expected %s, got '%s'", what, desc(t));
	return t;
}

static Tok *want_name(P *p)
{
	Tok *t = want(p, T_NAME, "name");
	for (int i = 0; KW[i]; i++)
		if (!strcmp(t->s, KW[i])) fail(p->f, p->file, t->line, "'%s' is a reserved word", t->s);
	return t;
}

static double snum(P *p)
{
	int neg = 0;
	if (isop(peek(p), "-")) next(p), neg = 1;
	Tok *t = want(p, T_NUM, "number");
	return neg ? -t->n : t->n;
}

static int posint(P *p)
{
	Tok *t = want(p, T_NUM, "integer");
	if (t->n < 1 || t->n != (double)(int)t->n || t->n > 1 << 24) fail(p->f, p->file, t->line, "expected positive integer, got '%s'", t->s);
	return (int)t->n;
}

static Sh type(P *p)
{
	Tok *t = next(p);
	if (!iskw(t, "f32")) fail(p->f, p->file, t->line, "expected type 'f32', got '%s'", desc(t));
	Sh s = { 0, { 0 } };
	if (isop(peek(p), "[")) {
		next(p);
		for (;;) {
			if (s.rank >= MAXRANK) fail(p->f, p->file, t->line, "rank exceeds %d", MAXRANK);
			s.dim[s.rank++] = posint(p);
			if (isop(peek(p), "]")) {
				next(p);
				break;
			}
			want_op(p, ",");
		}
	}
	return s;
}

static void init_add(P *p, Init *in, double v)
{
	if (in->nv == in->cap) {
		in->cap = in->cap ? 2 * in->cap : 16;
		double *nv = fa(p->f, (size_t)in->cap * sizeof *nv);
		if (in->nv) memcpy(nv, in->v, (size_t)in->nv * sizeof *nv);
		in->v = nv;
	}
	in->v[in->nv++] = v;
}

static void literal(P *p, Init *in)
{
	if (isop(peek(p), "[")) {
		next(p);
		for (;;) {
			literal(p, in);
			if (isop(peek(p), "]")) {
				next(p);
				return;
			}
			want_op(p, ",");
		}
	}
	init_add(p, in, snum(p));
}

static Init initializer(P *p)
{
	Tok *t = peek(p);
	Init in = { I_DATA, 0, t->line, 0, NULL, NULL };
	if (iskw(t, "zeros") || iskw(t, "ones")) {
		next(p);
		in.kind = iskw(t, "zeros") ? I_ZEROS : I_ONES;
	} else if (iskw(t, "fill")) {
		next(p);
		want_op(p, "(");
		in.kind = I_FILL;
		init_add(p, &in, snum(p));
		want_op(p, ")");
	} else if (iskw(t, "rand")) {
		next(p);
		want_op(p, "(");
		in.kind = I_RAND;
		init_add(p, &in, snum(p));
		want_op(p, ",");
		init_add(p, &in, snum(p));
		want_op(p, ")");
	} else if (iskw(t, "file")) {
		next(p);
		want_op(p, "(");
		in.kind = I_FILE;
		in.str = want(p, T_STR, "string")->s;
		want_op(p, ")");
	} else if (iskw(t, "env")) {
		next(p);
		want_op(p, "(");
		in.kind = I_ENV;
		in.str = want(p, T_STR, "string")->s;
		if (isop(peek(p), ",")) next(p), init_add(p, &in, snum(p));
		want_op(p, ")");
	} else {
		literal(p, &in);
	}
	return in;
}

static Ex *ex_new(P *p, int kind, int line)
{
	Ex *e = fa(p->f, sizeof *e);
	e->kind = kind;
	e->line = line;
	return e;
}

static void ex_arg(P *p, Ex *c, Ex *a)
{
	Ex **v = fa(p->f, (size_t)(c->nargs + 1) * sizeof *v);
	if (c->nargs) memcpy(v, c->args, (size_t)c->nargs * sizeof *v);
	v[c->nargs++] = a;
	c->args = v;
}

static Ex *call(P *p, const char *fn, Ex *a, Ex *b, int line)
{
	Ex *c = ex_new(p, E_CALL, line);
	c->name = fn;
	ex_arg(p, c, a);
	if (b) ex_arg(p, c, b);
	return c;
}

static Ex *expr(P *p);

static Ex *primary(P *p)
{
	Tok *t = next(p);
	if (t->k == T_NUM) {
		Ex *e = ex_new(p, E_NUM, t->line);
		e->num = t->n;
		return e;
	}
	if (isop(t, "(")) {
		Ex *e = expr(p);
		want_op(p, ")");
		return e;
	}
	if (t->k == T_NAME) {
		for (int i = 0; KW[i]; i++)
			if (!strcmp(t->s, KW[i])) fail(p->f, p->file, t->line, "unexpected keyword '%s' in expression", t->s);
		if (isop(peek(p), "(")) {
			next(p);
			Ex *c = ex_new(p, E_CALL, t->line);
			c->name = t->s;
			if (isop(peek(p), ")")) {
				next(p);
				return c;
			}
			for (;;) {
				ex_arg(p, c, expr(p));
				if (isop(peek(p), ")")) {
					next(p);
					return c;
				}
				want_op(p, ",");
			}
		}
		Ex *e = ex_new(p, E_REF, t->line);
		e->name = t->s;
		return e;
	}
	fail(p->f, p->file, t->line, "expected expression, got '%s'", desc(t));
	return NULL;
}

static Ex *unary(P *p)
{
	if (isop(peek(p), "-")) {
		int line = next(p)->line;
		Tok *t = peek(p);
		if (t->k == T_NUM) { /* a negative literal is one number */
			next(p);
			Ex *e = ex_new(p, E_NUM, line);
			e->num = -t->n;
			return e;
		}
		return call(p, "neg", unary(p), NULL, line);
	}
	return primary(p);
}

static Ex *term(P *p)
{
	Ex *e = unary(p);
	for (;;) {
		Tok *t = peek(p);
		const char *op = isop(t, "*") ? "mul" : isop(t, "/") ? "div" : isop(t, "@") ? "matmul" : NULL;
		if (!op) return e;
		next(p);
		e = call(p, op, e, unary(p), t->line);
	}
}

static Ex *expr(P *p)
{
	Ex *e = term(p);
	for (;;) {
		Tok *t = peek(p);
		const char *op = isop(t, "+") ? "add" : isop(t, "-") ? "sub" : NULL;
		if (!op) return e;
		next(p);
		e = call(p, op, e, term(p), t->line);
	}
}

static void block(P *p, St ***body, int *n, int *bline);

static const char **names_add(P *p, const char **a, int n, const char *s)
{
	const char **r = fa(p->f, (size_t)(n + 1) * sizeof *r);
	if (n) memcpy(r, a, (size_t)n * sizeof *r);
	r[n] = s;
	return r;
}

static St *stmt(P *p)
{
	Tok *t = peek(p);
	St *s = fa(p->f, sizeof *s);
	s->line = t->line;
	if (iskw(t, "return")) {
		next(p);
		s->kind = S_RETURN;
		s->e = expr(p);
		want(p, T_NL, "end of line");
	} else if (iskw(t, "train")) { /* parsed for its diagnostics; lowering refuses it */
		next(p);
		s->kind = S_TRAIN;
		s->e = expr(p);
		if (iskw(peek(p), "with")) {
			next(p);
			want(p, T_NAME, "optimizer name");
			if (isop(peek(p), "(")) {
				next(p);
				for (;;) {
					want(p, T_NAME, "option name");
					want_op(p, "=");
					snum(p);
					if (isop(peek(p), ")")) {
						next(p);
						break;
					}
					want_op(p, ",");
				}
			}
		}
		if (iskw(peek(p), "over")) {
			next(p);
			for (;;) {
				want_name(p);
				if (!isop(peek(p), ",")) break;
				next(p);
			}
		}
		want(p, T_NL, "end of line");
	} else if (iskw(t, "update")) {
		next(p);
		s->kind = S_UPDATE;
		s->name = want_name(p)->s;
		if (isop(peek(p), "[")) {
			next(p);
			s->rows = expr(p);
			want_op(p, "]");
		}
		want_op(p, "=");
		s->e = expr(p);
		want(p, T_NL, "end of line");
	} else if (iskw(t, "scan")) {
		next(p);
		s->kind = S_SCAN;
		for (;;) {
			Tok *n = want_name(p);
			s->cs = names_add(p, s->cs, s->ncs++, n->s);
			if (!isop(peek(p), ",")) break;
			next(p);
		}
		Tok *o = next(p);
		if (!iskw(o, "over")) fail(p->f, p->file, o->line, "expected 'over' after the scan carries, got '%s'", desc(o));
		for (;;) {
			Tok *n = want_name(p);
			Tok *in = next(p);
			if (!iskw(in, "in")) fail(p->f, p->file, in->line, "expected 'in' after scan slice '%s', got '%s'", n->s, desc(in));
			Ex *e = expr(p);
			Ex **xe = fa(p->f, (size_t)(s->nx + 1) * sizeof *xe);
			if (s->nx) memcpy(xe, s->xe, (size_t)s->nx * sizeof *xe);
			xe[s->nx] = e;
			s->xe = xe;
			s->xn = names_add(p, s->xn, s->nx++, n->s);
			if (!isop(peek(p), ",")) break;
			next(p);
		}
		want_op(p, ":");
		block(p, &s->body, &s->nbody, &s->bline);
	} else if (iskw(t, "emit")) {
		next(p);
		s->kind = S_EMIT;
		s->name = want_name(p)->s;
		want_op(p, "=");
		s->e = expr(p);
		want(p, T_NL, "end of line");
	} else if (iskw(t, "think")) {
		next(p);
		s->kind = S_THINK;
		s->name = want_name(p)->s;
		Tok *fo = next(p);
		if (!iskw(fo, "for")) fail(p->f, p->file, fo->line, "expected 'for' after think state, got '%s'", desc(fo));
		s->maxit = posint(p);
		s->eps = -1;
		if (iskw(peek(p), "until")) {
			next(p);
			s->eps = snum(p);
			if (s->eps < 0) fail(p->f, p->file, s->line, "halting threshold must be >= 0");
		} else if (iskw(peek(p), "halt")) {
			next(p);
			s->has_halt = 1;
			s->halt = want_name(p)->s;
			s->hthr = 0.5;
			if (iskw(peek(p), "at")) {
				next(p);
				s->hthr = snum(p);
				if (s->hthr <= 0 || s->hthr >= 1) fail(p->f, p->file, s->line, "halting threshold must be in (0, 1)");
			}
		}
		want_op(p, ":");
		block(p, &s->body, &s->nbody, &s->bline);
	} else {
		s->kind = S_SET;
		s->name = want_name(p)->s;
		want_op(p, "=");
		s->e = expr(p);
		want(p, T_NL, "end of line");
	}
	return s;
}

static void block(P *p, St ***body, int *n, int *bline)
{
	want(p, T_NL, "end of line");
	*bline = want(p, T_INDENT, "indented block")->line;
	*body = NULL;
	*n = 0;
	while (peek(p)->k != T_DEDENT && peek(p)->k != T_EOF) {
		St *s = stmt(p);
		St **v = fa(p->f, (size_t)(*n + 1) * sizeof *v);
		if (*n) memcpy(v, *body, (size_t)*n * sizeof *v);
		v[(*n)++] = s;
		*body = v;
	}
	want(p, T_DEDENT, "dedent");
}

static Decl *decl(P *p)
{
	Tok *t = next(p);
	Decl *d = fa(p->f, sizeof *d);
	d->line = t->line;
	if (iskw(t, "import")) {
		d->kind = D_IMPORT;
		d->str = want(p, T_STR, "import path string")->s;
		want(p, T_NL, "end of line");
	} else if (iskw(t, "model")) {
		d->kind = D_MODEL;
		d->name = want_name(p)->s;
		want(p, T_NL, "end of line");
	} else if (iskw(t, "param") || iskw(t, "state")) {
		d->kind = iskw(t, "param") ? D_PARAM : D_STATE;
		d->name = want_name(p)->s;
		want_op(p, ":");
		d->sh = type(p);
		want_op(p, "=");
		d->init = initializer(p);
		want(p, T_NL, "end of line");
	} else if (iskw(t, "def")) {
		d->kind = D_DEF;
		d->name = want_name(p)->s;
		want_op(p, "(");
		if (!isop(peek(p), ")")) {
			for (;;) {
				Tok *a = want_name(p);
				want_op(p, ":");
				Sh sh = type(p);
				Sh *as = fa(p->f, (size_t)(d->nargs + 1) * sizeof *as);
				if (d->nargs) memcpy(as, d->as, (size_t)d->nargs * sizeof *as);
				as[d->nargs] = sh;
				d->as = as;
				d->an = names_add(p, d->an, d->nargs++, a->s);
				if (isop(peek(p), ")")) break;
				want_op(p, ",");
			}
		}
		want_op(p, ")");
		want_op(p, "->");
		d->sh = type(p);
		want_op(p, ":");
		block(p, &d->body, &d->nbody, &d->bline);
	} else {
		fail(p->f, p->file, d->line, "expected 'import', 'model', 'param', 'state' or 'def', got '%s'", desc(t));
	}
	return d;
}

/* ------------------------------------------------------------- files --- */

typedef struct {
	Decl **d;
	int n;
	const char **seen;
	int nseen;
} Prog;

static char *read_all(F *f, const char *path, size_t *len)
{
	FILE *fp = fopen(path, "rb");
	if (!fp) return NULL;
	size_t cap = 4096, n = 0;
	char *buf = malloc(cap);
	for (;;) {
		if (!buf) break;
		if (n + 4096 > cap) {
			char *nb = realloc(buf, cap *= 2);
			if (!nb) {
				free(buf);
				buf = NULL;
				break;
			}
			buf = nb;
		}
		size_t k = fread(buf + n, 1, 4096, fp);
		n += k;
		if (k < 4096) break;
	}
	fclose(fp);
	if (!buf) fail(f, NULL, 0, "out of memory");
	char *r = fstr(f, buf, n);
	free(buf);
	if (len) *len = n;
	return r;
}

static char *dir_of(F *f, const char *path)
{
	const char *sl = strrchr(path, '/');
	return sl ? fstr(f, path, (size_t)(sl - path)) : fstr(f, ".", 1);
}

static char *join(F *f, const char *dir, const char *rel)
{
	if (rel[0] == '/') return fstr(f, rel, strlen(rel));
	char *r = fa(f, strlen(dir) + strlen(rel) + 2);
	sprintf(r, "%s/%s", dir, rel);
	return r;
}

static void load_file(F *f, Prog *g, const char *path, int depth, int root, const char *importer, int iline)
{
	if (depth > 64) fail(f, importer, iline, "import nesting too deep (cycle involving '%s'?)", path);
	for (int i = 0; i < g->nseen; i++)
		if (!strcmp(g->seen[i], path)) return; /* merged already */
	const char **seen = fa(f, (size_t)(g->nseen + 1) * sizeof *seen);
	if (g->nseen) memcpy(seen, g->seen, (size_t)g->nseen * sizeof *seen);
	seen[g->nseen++] = path;
	g->seen = seen;
	char *src = read_all(f, path, NULL);
	if (!src) {
		if (importer) fail(f, importer, iline, "cannot open import '%s'", path);
		fail(f, NULL, 0, "cannot open '%s'", path);
	}
	P p = { f, path, NULL, 0, 0, 0 };
	lex(&p, src);
	for (;;) {
		Tok *t = peek(&p);
		if (t->k == T_EOF) break;
		if (t->k == T_NL) {
			next(&p);
			continue;
		}
		if (t->k == T_INDENT) fail(f, path, t->line, "unexpected indent");
		Decl *d = decl(&p);
		int keep = root || d->kind == D_PARAM || d->kind == D_STATE || (d->kind == D_DEF && strcmp(d->name, "forward"));
		if (d->kind == D_IMPORT) {
			load_file(f, g, join(f, dir_of(f, path), d->str), depth + 1, 0, path, d->line);
		} else if (keep) {
			Decl **v = fa(f, (size_t)(g->n + 1) * sizeof *v);
			if (g->n) memcpy(v, g->d, (size_t)g->n * sizeof *v);
			v[g->n++] = d;
			g->d = v;
		}
	}
}

/* ---------------------------------------------------------- lowering --- */

typedef struct {
	const char **name;
	int *val, n;
} Env;

typedef struct Emits {
	int level;
	const char **name;
	int *val, n;
} Emits;

typedef struct {
	F *f;
	const char *file;
	Prog *g;
	Env globals;
	int depth, in_loop;
	const char *loop_kw;
	Emits *emits;
} L;

static int env_get(const Env *e, const char *n)
{
	for (int i = e->n - 1; i >= 0; i--)
		if (!strcmp(e->name[i], n)) return e->val[i];
	return -1;
}

static void env_set(F *f, Env *e, const char *n, int v)
{
	for (int i = e->n - 1; i >= 0; i--)
		if (!strcmp(e->name[i], n)) {
			e->val[i] = v;
			return;
		}
	const char **nn = fa(f, (size_t)(e->n + 1) * sizeof *nn);
	int *nv = fa(f, (size_t)(e->n + 1) * sizeof *nv);
	if (e->n) memcpy(nn, e->name, (size_t)e->n * sizeof *nn), memcpy(nv, e->val, (size_t)e->n * sizeof *nv);
	nn[e->n] = n;
	nv[e->n++] = v;
	e->name = nn;
	e->val = nv;
}

static Env env_copy(F *f, const Env *e)
{
	Env c = { fa(f, (size_t)(e->n + 1) * sizeof(char *)), fa(f, (size_t)(e->n + 1) * sizeof(int)), e->n };
	if (e->n) memcpy(c.name, e->name, (size_t)e->n * sizeof *c.name), memcpy(c.val, e->val, (size_t)e->n * sizeof *c.val);
	return c;
}

static Decl *find_def(L *l, const char *n)
{
	for (int i = 0; i < l->g->n; i++)
		if (l->g->d[i]->kind == D_DEF && !strcmp(l->g->d[i]->name, n)) return l->g->d[i];
	return NULL;
}

/* an instruction of a table operation on existing values; die() wording per caller */
static int op_emit(L *l, Blk *b, int op, const int *args, int na, int line, const char *prefix)
{
	F *f = l->f;
	Sh in[3], out;
	char err[320];
	for (int i = 0; i < na && i < 3; i++) in[i] = f->val[args[i]].sh;
	if (infer(op, in, na, &out, err)) fail(f, l->file, line, "%s%s", prefix, err);
	int o = newval(f, K_TMP, &out, NULL);
	int i = push(f, b);
	Ins *ins = &b->v[i];
	ins->op = op;
	ins->out = o;
	ins->na = na;
	for (int j = 0; j < na; j++) ins->a[j] = args[j];
	return o;
}

static int op2(L *l, Blk *b, const char *name, int p, int q, int line) /* the reference's generated-code helper */
{
	int args[2] = { p, q };
	return op_emit(l, b, op_id(name), args, q >= 0 ? 2 : 1, line, "autodiff: ");
}

static int konst(L *l, Blk *b, float k)
{
	Sh s = { 0, { 0 } };
	int o = newval(l->f, K_TMP, &s, NULL);
	int i = push(l->f, b);
	b->v[i].op = op_id("const");
	b->v[i].out = o;
	b->v[i].k = k;
	return o;
}

static int reshape_to(L *l, Blk *b, int x, const Sh *to)
{
	int o = newval(l->f, K_TMP, to, NULL);
	int i = push(l->f, b);
	b->v[i].op = op_id("reshape");
	b->v[i].out = o;
	b->v[i].na = 1;
	b->v[i].a[0] = x;
	return o;
}

/* a compiler-generated constant param, shared by name */
static int const_param(L *l, const char *name, const Sh *sh, const float *data)
{
	F *f = l->f;
	for (int v = 0; v < f->nval; v++)
		if (f->val[v].kind == K_PARAM && f->val[v].name && !strcmp(f->val[v].name, name)) return v;
	int v = newval(f, K_PARAM, sh, fstr(f, name, strlen(name)));
	int n = numel(sh);
	f->val[v].data = fa(f, (size_t)n * sizeof(float));
	memcpy(f->val[v].data, data, (size_t)n * sizeof(float));
	return v;
}

static int lower_expr(L *l, Blk *b, Env *e, Ex *x);
static int lower_block(L *l, Blk *b, Env *e, St **body, int n, int is_fn, int line);

static int lookup(L *l, Env *e, const char *n, int line)
{
	int v = env_get(e, n);
	if (v < 0) v = env_get(&l->globals, n);
	if (v < 0) fail(l->f, l->file, line, "undefined name '%s'", n);
	return v;
}

static int is_num(const Ex *x) { return x->kind == E_NUM; }

/* rope(x, pos) and attention(Q, K, V, W): expansions into table ops (src/lower.c:370-419) */
static int lower_attn(L *l, Blk *b, Env *e, Ex *x)
{
	F *f = l->f;
	char name[64], s0[64];
	int line = x->line;
	if (!strcmp(x->name, "rope")) {
		if (x->nargs != 2) fail(f, l->file, line, "'rope' takes (x, position)");
		int v = lower_expr(l, b, e, x->args[0]), p = lower_expr(l, b, e, x->args[1]);
		Sh xs = f->val[v].sh, ps = f->val[p].sh;
		int d = xs.dim[xs.rank - 1];
		int ok = (xs.rank == 1 && ps.rank == 0) || (xs.rank == 2 && ps.rank == 1 && ps.dim[0] == xs.dim[0]);
		if (!ok || d % 2) fail(f, l->file, line, "'rope' takes x (d) with a scalar position or x (T, d) with positions (T), d even");
		float *fr = fa(f, (size_t)d * sizeof *fr), *sw = fa(f, (size_t)d * (size_t)d * sizeof *sw);
		for (int i = 0; i < d; i++) fr[i] = (float)pow(10000.0, -(double)(i / 2 * 2) / d);
		for (int i = 0; i < d; i += 2) sw[i * d + i + 1] = 1, sw[(i + 1) * d + i] = -1;
		Sh s1 = { 1, { d } }, s2 = { 2, { d, d } };
		snprintf(name, sizeof name, "__rope_freq_%d", d);
		int fv = const_param(l, name, &s1, fr);
		snprintf(name, sizeof name, "__swap_%d", d);
		int sv = const_param(l, name, &s2, sw);
		int ang = xs.rank == 1 ? op2(l, b, "mul", fv, p, line) : op2(l, b, "outer", p, fv, line);
		/* x cos(a) + (x @ swap) sin(a), instructions in the reference's order (the sine term first) */
		int sn = op2(l, b, "sin", ang, -1, line);
		int xs_ = op2(l, b, "matmul", v, sv, line);
		int st = op2(l, b, "mul", xs_, sn, line);
		int cs = op2(l, b, "cos", ang, -1, line);
		int ct = op2(l, b, "mul", v, cs, line);
		return op2(l, b, "add", ct, st, line);
	}
	(void)s0;
	if (x->nargs != 4) fail(f, l->file, line, "'attention' takes (Q, K, V, window)");
	Ex *wd = x->args[3];
	if (!is_num(wd) || wd->num < 1 || wd->num != (double)(int)wd->num) fail(f, l->file, line, "'attention' window must be a positive integer literal");
	int W = (int)wd->num;
	int q = lower_expr(l, b, e, x->args[0]), k = lower_expr(l, b, e, x->args[1]), v = lower_expr(l, b, e, x->args[2]);
	Sh qs = f->val[q].sh, ks = f->val[k].sh, vs = f->val[v].sh;
	if (qs.rank != 2 || !sheq(&qs, &ks) || vs.rank != 2 || vs.dim[0] != qs.dim[0])
		fail(f, l->file, line, "'attention' needs Q and K of one shape (T, d) and V (T, e)");
	int T = qs.dim[0];
	float *mk = fa(f, (size_t)T * (size_t)T * sizeof *mk);
	for (int t = 0; t < T; t++)
		for (int s = 0; s < T; s++) mk[t * T + s] = s <= t && t - s < W ? 0.0f : -1e9f;
	Sh ms = { 2, { T, T } };
	snprintf(name, sizeof name, "__causal_%d_%d", T, W);
	int mv = const_param(l, name, &ms, mk);
	int sk = konst(l, b, (float)(1.0 / sqrt((double)qs.dim[1]))); /* the scale's const precedes the product */
	int kt = op2(l, b, "transpose", k, -1, line);
	int sc = op2(l, b, "mul", op2(l, b, "matmul", q, kt, line), sk, line);
	sc = op2(l, b, "add", sc, mv, line);
	return op2(l, b, "matmul", op2(l, b, "softmax", sc, -1, line), v, line);
}

/* take_along(x, i): the gather along the last axis as one take over the flattened rows (src/lower.c:326-364) */
static int lower_take_along(L *l, Blk *b, Env *e, Ex *x)
{
	F *f = l->f;
	int line = x->line;
	char s0[64], s1[64], name[64];
	if (x->nargs != 2) fail(f, l->file, line, "'take_along' takes (x, indices)");
	int v = lower_expr(l, b, e, x->args[0]), iv = lower_expr(l, b, e, x->args[1]);
	Sh xs = f->val[v].sh, is = f->val[iv].sh;
	int ok = xs.rank >= 1 && is.rank == xs.rank;
	for (int d = 0; ok && d < xs.rank - 1; d++) ok = xs.dim[d] == is.dim[d];
	if (!ok)
		fail(f, l->file, line, "'take_along' needs x (..., n) and indices (..., k) with the same leading dimensions; got %s and %s",
		     shstr(&xs, s0), shstr(&is, s1));
	int n = xs.dim[xs.rank - 1], k = is.dim[is.rank - 1], R = numel(&xs) / n;
	/* in range: step(i + 1) * step(n - i); the second factor's instructions come first */
	int hi = op2(l, b, "step", op2(l, b, "sub", konst(l, b, (float)n), iv, line), -1, line);
	int k1 = konst(l, b, 1);
	int lo = op2(l, b, "step", op2(l, b, "add", iv, k1, line), -1, line);
	int okm = op2(l, b, "mul", lo, hi, line);
	int sh = iv;
	if (R > 1) {
		float *off = fa(f, (size_t)R * sizeof *off);
		for (int r = 0; r < R; r++) off[r] = (float)r * (float)n;
		Sh os = { 2, { R, 1 } }, is2 = { 2, { R, k } };
		snprintf(name, sizeof name, "__rowoff_%d_%d", R, n);
		int ov = const_param(l, name, &os, off);
		sh = op2(l, b, "add", reshape_to(l, b, iv, &is2), ov, line);
		okm = reshape_to(l, b, okm, &is2);
	}
	int one = konst(l, b, 1);
	int idx = op2(l, b, "sub", op2(l, b, "add", op2(l, b, "mul", sh, okm, line), okm, line), one, line);
	Sh fl = { 2, { R * n, 1 } }, il = { 1, { R * k } };
	int ri = reshape_to(l, b, idx, &il);
	int rv = reshape_to(l, b, v, &fl);
	int g = op2(l, b, "take", rv, ri, line);
	return reshape_to(l, b, g, &is);
}

static int lower_expr(L *l, Blk *b, Env *e, Ex *x)
{
	F *f = l->f;
	char s0[64], s1[64];
	if (x->kind == E_NUM) return konst(l, b, (float)x->num);
	if (x->kind == E_REF) return lookup(l, e, x->name, x->line);
	const char *fn = x->name;
	if (!strcmp(fn, "grad")) fail(f, l->file, x->line, "'grad' (automatic differentiation) is not part of the batch backend's front end");
	if (!strcmp(fn, "rope") || !strcmp(fn, "attention")) return lower_attn(l, b, e, x);
	if (!strcmp(fn, "topk") || !strcmp(fn, "memory_scan") || !strcmp(fn, "memory_final") || !strcmp(fn, "suffix_match"))
		fail(f, l->file, x->line, "'%s' is not run by the batch backend", fn);
	if (!strcmp(fn, "take_along")) return lower_take_along(l, b, e, x);
	if (!strcmp(fn, "reshape")) {
		Sh to = { 0, { 0 } };
		if (x->nargs < 2 || x->nargs - 1 > MAXRANK) fail(f, l->file, x->line, "'reshape' takes a tensor and 1 to %d dimensions", MAXRANK);
		for (int i = 1; i < x->nargs; i++) {
			Ex *d = x->args[i];
			if (!is_num(d) || d->num < 1 || d->num != (double)(int)d->num)
				fail(f, l->file, x->line, "'reshape' dimensions must be positive integer literals");
			to.dim[to.rank++] = (int)d->num;
		}
		int v = lower_expr(l, b, e, x->args[0]);
		if (numel(&to) != numel(&f->val[v].sh))
			fail(f, l->file, x->line, "'reshape' from %s to %s changes the element count", shstr(&f->val[v].sh, s0), shstr(&to, s1));
		return reshape_to(l, b, v, &to);
	}
	int na = x->nargs, args[16];
	if (na > 16) fail(f, l->file, x->line, "too many arguments");
	for (int i = 0; i < na; i++) args[i] = lower_expr(l, b, e, x->args[i]);
	Decl *def = find_def(l, fn);
	if (def) { /* inline the def with its arguments bound */
		if (def->nargs != na) fail(f, l->file, x->line, "'%s' takes %d argument(s), got %d", fn, def->nargs, na);
		if (++l->depth > 64) fail(f, l->file, x->line, "inlining depth exceeded (recursive def '%s'?)", fn);
		Env fe = { 0 };
		for (int i = 0; i < na; i++) {
			if (!sheq(&def->as[i], &f->val[args[i]].sh))
				fail(f, l->file, x->line, "argument %d of '%s': expected %s, got %s", i + 1, fn, shstr(&def->as[i], s0), shstr(&f->val[args[i]].sh, s1));
			env_set(f, &fe, def->an[i], args[i]);
		}
		int r = lower_block(l, b, &fe, def->body, def->nbody, 1, def->bline);
		if (!sheq(&def->sh, &f->val[r].sh))
			fail(f, l->file, def->line, "'%s' declared to return %s, returns %s", fn, shstr(&def->sh, s0), shstr(&f->val[r].sh, s1));
		l->depth--;
		return r;
	}
	if (!strcmp(fn, "mse") || !strcmp(fn, "bce") || !strcmp(fn, "xent")) {
		if (na != 2) fail(f, l->file, x->line, "'%s' takes (prediction, target)", fn);
		if (!sheq(&f->val[args[0]].sh, &f->val[args[1]].sh))
			fail(f, l->file, x->line, "'%s' prediction %s and target %s differ in shape", fn, shstr(&f->val[args[0]].sh, s0), shstr(&f->val[args[1]].sh, s1));
		int p = args[0], t = args[1], ln = x->line;
		if (!strcmp(fn, "mse")) {
			int d = op2(l, b, "sub", p, t, ln);
			return op2(l, b, "mean", op2(l, b, "mul", d, d, ln), -1, ln);
		}
		if (!strcmp(fn, "bce")) { /* -mean(t log(p + 1e-7) + (1 - t) log(1 - p + 1e-7)), in the reference's instruction order */
			int lp = op2(l, b, "log", op2(l, b, "add", p, konst(l, b, 1e-7f), ln), -1, ln);
			int e7 = konst(l, b, 1e-7f);
			int lq = op2(l, b, "log", op2(l, b, "add", op2(l, b, "sub", konst(l, b, 1), p, ln), e7, ln), -1, ln);
			int qt = op2(l, b, "mul", op2(l, b, "sub", konst(l, b, 1), t, ln), lq, ln);
			int pt = op2(l, b, "mul", t, lp, ln);
			int s = op2(l, b, "add", pt, qt, ln);
			return op2(l, b, "neg", op2(l, b, "mean", s, -1, ln), -1, ln);
		}
		int rk = f->val[p].sh.rank;
		if (rk != 1 && rk != 2) fail(f, l->file, x->line, "'xent' needs logits of shape (C) or a batch (B, C), with one-hot targets");
		int e12 = konst(l, b, 1e-12f); /* -sum(t log(softmax(p) + 1e-12)), averaged over a batch's rows */
		int ls = op2(l, b, "log", op2(l, b, "add", op2(l, b, "softmax", p, -1, ln), e12, ln), -1, ln);
		int s = op2(l, b, "sum", op2(l, b, "mul", t, ls, ln), -1, ln);
		if (rk == 2) s = op2(l, b, "div", s, konst(l, b, (float)f->val[p].sh.dim[0]), ln);
		return op2(l, b, "neg", s, -1, ln);
	}
	int op = op_of(!strcmp(fn, "dot") ? "matmul" : fn);
	if (op < 0) fail(f, l->file, x->line, "unknown function '%s'", fn);
	if (OPS[op].cls == C_OTHER) fail(f, l->file, x->line, "'%s' is not run by the batch backend", fn);
	if (na != OPS[op].arity) fail(f, l->file, x->line, "'%s' takes %d operand(s), got %d", OPS[op].name, OPS[op].arity, na);
	return op_emit(l, b, op, args, na, x->line, "");
}

/* scan C, ... over X in E, ...: body (src/lower.c:420-527) */
static void lower_scan(L *l, Blk *b, Env *e, St *s)
{
	F *f = l->f;
	char s0[64], s1[64];
	int T = -1, nc = s->ncs, nx = s->nx;
	int *seq = fa(f, (size_t)(nx + 1) * sizeof *seq);
	for (int j = 0; j < nx; j++) {
		seq[j] = lower_expr(l, b, e, s->xe[j]);
		const Sh *q = &f->val[seq[j]].sh;
		if (q->rank < 1) fail(f, l->file, s->line, "scan sequence '%s' must have rank >= 1 (steps along the first axis)", s->xn[j]);
		if (T >= 0 && q->dim[0] != T) fail(f, l->file, s->line, "scan sequences differ in length: %d and %d steps", T, q->dim[0]);
		T = q->dim[0];
	}
	int *c = fa(f, (size_t)(nc + 1) * sizeof *c), *ci = fa(f, (size_t)(nc + 1) * sizeof *ci), *cn = fa(f, (size_t)(nc + 1) * sizeof *cn);
	int *xt = fa(f, (size_t)(nx + 1) * sizeof *xt);
	for (int k = 0; k < nc; k++) {
		const char *n = s->cs[k];
		for (int j = 0; j < k; j++)
			if (!strcmp(s->cs[j], n)) fail(f, l->file, s->line, "scan carry '%s' listed twice", n);
		int init = env_get(e, n);
		if (init < 0) {
			if (env_get(&l->globals, n) >= 0) fail(f, l->file, s->line, "scan carry '%s' is a parameter", n);
			fail(f, l->file, s->line, "scan carry '%s' must be assigned before the loop", n);
		}
		Sh sh = f->val[init].sh;
		c[k] = newval(f, K_TMP, &sh, NULL);
		ci[k] = init;
		cn[k] = -1;
	}
	for (int j = 0; j < nx; j++) {
		Sh q = f->val[seq[j]].sh;
		for (int d = 1; d < q.rank; d++) q.dim[d - 1] = q.dim[d];
		q.rank--;
		xt[j] = newval(f, K_TMP, &q, NULL);
	}
	int idx = push(f, b);
	Blk *body = fa(f, sizeof *body);
	Env inner = env_copy(f, e);
	for (int k = 0; k < nc; k++) env_set(f, &inner, s->cs[k], c[k]);
	for (int j = 0; j < nx; j++) env_set(f, &inner, s->xn[j], xt[j]);
	int outer_n = e->n;
	const char *kw = l->loop_kw;
	Emits em = { l->in_loop + 1, NULL, NULL, 0 }, *save = l->emits;
	l->loop_kw = "scan";
	l->in_loop++;
	l->emits = &em;
	lower_block(l, body, &inner, s->body, s->nbody, 0, s->line);
	l->in_loop--;
	l->loop_kw = kw;
	l->emits = save;
	for (int j = 0; j < outer_n; j++) {
		const char *n = e->name[j];
		int carried = 0;
		for (int k = 0; k < nc; k++) carried |= !strcmp(n, s->cs[k]);
		for (int j2 = 0; j2 < nx; j2++) carried |= !strcmp(n, s->xn[j2]);
		if (!carried && inner.val[j] != e->val[j])
			fail(f, l->file, s->line, "scan block assigns outer variable '%s'; only the carries are carried (use emit to collect per-step values)", n);
	}
	for (int k = 0; k < nc; k++) {
		int nv = env_get(&inner, s->cs[k]);
		if (!sheq(&f->val[nv].sh, &f->val[c[k]].sh))
			fail(f, l->file, s->line, "scan carry '%s' changes shape from %s to %s", s->cs[k], shstr(&f->val[c[k]].sh, s0), shstr(&f->val[nv].sh, s1));
		for (int j = 0; j < nc; j++) /* another carry's value: a copy, so carries can advance in any order */
			if (j != k && nv == c[j]) nv = op2(l, body, "mul", nv, konst(l, body, 1), s->line);
		cn[k] = nv;
	}
	int *y = fa(f, (size_t)(em.n + 1) * sizeof *y), *ys = fa(f, (size_t)(em.n + 1) * sizeof *ys);
	for (int i = 0; i < em.n; i++) {
		Sh q = f->val[em.val[i]].sh;
		if (q.rank == MAXRANK) fail(f, l->file, s->line, "emit '%s': a stack of rank-%d values exceeds rank %d", em.name[i], q.rank, MAXRANK);
		for (int d = q.rank; d > 0; d--) q.dim[d] = q.dim[d - 1];
		q.dim[0] = T;
		q.rank++;
		y[i] = em.val[i];
		ys[i] = newval(f, K_TMP, &q, NULL);
	}
	Ins *in = &b->v[idx];
	in->op = op_id("scan");
	in->T = T;
	in->nc = nc, in->c = c, in->cinit = ci, in->cnext = cn;
	in->nx = nx, in->x = seq, in->xt = xt;
	in->ny = em.n, in->y = y, in->ys = ys;
	in->out = nc ? c[0] : -1;
	in->body = body;
	for (int k = 0; k < nc; k++) env_set(f, e, s->cs[k], c[k]);
	for (int i = 0; i < em.n; i++) env_set(f, e, em.name[i], ys[i]);
}

static int lower_block(L *l, Blk *b, Env *e, St **body, int n, int is_fn, int line)
{
	F *f = l->f;
	char s0[64], s1[64], s2[64];
	for (int i = 0; i < n; i++) {
		St *s = body[i];
		switch (s->kind) {
		case S_RETURN:
			if (!is_fn) fail(f, l->file, s->line, "'return' inside %s block", l->loop_kw);
			if (i != n - 1) fail(f, l->file, body[i + 1]->line, "unreachable statement after return");
			return lower_expr(l, b, e, s->e);
		case S_SET: {
			int v = lower_expr(l, b, e, s->e);
			int g = env_get(&l->globals, s->name);
			if (g >= 0 && f->val[g].kind == K_STATE) fail(f, l->file, s->line, "cannot assign to state '%s'; use 'update %s = ...'", s->name, s->name);
			if (g >= 0) fail(f, l->file, s->line, "cannot assign to parameter '%s'", s->name);
			env_set(f, e, s->name, v);
			break;
		}
		case S_TRAIN:
			fail(f, l->file, s->line, "'train' (training) is not part of the batch backend's front end");
			break;
		case S_UPDATE: {
			if (l->depth > 0) fail(f, l->file, s->line, "'update' is only allowed in the body of 'forward', not in a def");
			if (l->in_loop) fail(f, l->file, s->line, "'update' inside %s block (a state changes once per run)", l->loop_kw);
			int sv = env_get(&l->globals, s->name);
			if (sv >= 0 && f->val[sv].kind == K_PARAM) fail(f, l->file, s->line, "'%s' is a read-only param; declare it with 'state' to update it", s->name);
			if (sv < 0 || f->val[sv].kind != K_STATE) fail(f, l->file, s->line, "'%s' is not a state", s->name);
			for (int k = 0; k < f->nupd; k++)
				if (f->ust[k] == sv) fail(f, l->file, s->line, "state '%s' updated twice in one run", s->name);
			int rows = s->rows ? lower_expr(l, b, e, s->rows) : -1;
			int v = lower_expr(l, b, e, s->e);
			const Sh *st = &f->val[sv].sh, *sr = &f->val[v].sh;
			if (rows < 0) {
				if (!sheq(st, sr)) fail(f, l->file, s->line, "update of state '%s' %s with a value of shape %s", s->name, shstr(st, s0), shstr(sr, s1));
			} else {
				const Sh *ri = &f->val[rows].sh;
				int ok = st->rank >= 1 && ri->rank == 1 && sr->rank == st->rank && sr->dim[0] == ri->dim[0];
				for (int d = 1; ok && d < st->rank; d++) ok = sr->dim[d] == st->dim[d];
				if (!ok)
					fail(f, l->file, s->line,
					     "row update of state '%s' %s needs rows (n) and a value (n, ...) matching its trailing dimensions; got rows %s and value %s",
					     s->name, shstr(st, s0), shstr(ri, s2), shstr(sr, s1));
			}
			f->ust = ints_add(f, f->ust, f->nupd, sv);
			f->usrc = ints_add(f, f->usrc, f->nupd, v);
			f->urows = ints_add(f, f->urows, f->nupd, rows);
			f->nupd++;
			break;
		}
		case S_THINK: {
			int init = env_get(e, s->name);
			if (init < 0) {
				if (env_get(&l->globals, s->name) >= 0) fail(f, l->file, s->line, "think state '%s' is a parameter", s->name);
				fail(f, l->file, s->line, "think state '%s' must be assigned before the loop", s->name);
			}
			Sh sh = f->val[init].sh;
			int state = newval(f, K_TMP, &sh, NULL);
			int idx = push(f, b);
			Blk *tb = fa(f, sizeof *tb);
			Env inner = env_copy(f, e);
			env_set(f, &inner, s->name, state);
			int outer_n = e->n;
			const char *kw = l->loop_kw;
			l->loop_kw = "think";
			l->in_loop++;
			lower_block(l, tb, &inner, s->body, s->nbody, 0, s->line);
			l->in_loop--;
			l->loop_kw = kw;
			for (int j = 0; j < outer_n; j++)
				if (strcmp(e->name[j], s->name) && inner.val[j] != e->val[j])
					fail(f, l->file, s->line, "think block assigns outer variable '%s'; only the state '%s' is carried", e->name[j], s->name);
			int yv = env_get(&inner, s->name), hv = -1;
			if (s->has_halt) {
				hv = env_get(&inner, s->halt);
				if (hv < 0) fail(f, l->file, s->line, "halting value '%s' is not defined in the think body", s->halt);
				if (f->val[hv].sh.rank != 0) fail(f, l->file, s->line, "halting value '%s' must be a scalar probability", s->halt);
			}
			Ins *in = &b->v[idx];
			in->op = op_id("think");
			in->out = state;
			in->init = init;
			in->maxit = s->maxit;
			in->eps = (float)s->eps;
			in->body = tb;
			in->yield = yv;
			in->halt = hv;
			in->hthr = s->has_halt ? (float)s->hthr : 0.5f;
			env_set(f, e, s->name, state);
			break;
		}
		case S_EMIT: {
			Emits *em = l->emits;
			if (!em || em->level != l->in_loop) fail(f, l->file, s->line, "'emit' is only allowed directly in a scan body");
			for (int k = 0; k < em->n; k++)
				if (!strcmp(em->name[k], s->name)) fail(f, l->file, s->line, "'%s' emitted twice in one scan", s->name);
			int v = lower_expr(l, b, e, s->e);
			const char **nn = fa(f, (size_t)(em->n + 1) * sizeof *nn);
			if (em->n) memcpy(nn, em->name, (size_t)em->n * sizeof *nn);
			nn[em->n] = s->name;
			em->name = nn;
			em->val = ints_add(f, em->val, em->n, v);
			em->n++;
			break;
		}
		case S_SCAN:
			lower_scan(l, b, e, s);
			break;
		}
	}
	if (is_fn) fail(f, l->file, line, "function body has no 'return'");
	return -1;
}

static uint32_t xorshift(uint32_t *s)
{
	uint32_t x = *s;
	x ^= x << 13;
	x ^= x >> 17;
	x ^= x << 5;
	return *s = x;
}

/* env("NAME") values: numbers separated by blanks or commas, to '#' (src/io.c:25-41) */
static int parse_row(const char *s, float *v, int max, const char **bad)
{
	int n = 0;
	for (;;) {
		while (*s == ' ' || *s == '\t' || *s == ',' || *s == '\r' || *s == '\n') s++;
		if (!*s || *s == '#') return n;
		char *e;
		float x = strtof(s, &e);
		if (e == s || (*e && !strchr(" \t,\r\n#", *e))) {
			*bad = s;
			return -1;
		}
		if (n < max) v[n] = x;
		n++;
		s = e;
	}
}

static float *materialize(L *l, const Init *in, const Sh *sh, const char *pname)
{
	F *f = l->f;
	int n = numel(sh);
	float *d = fa(f, (size_t)n * sizeof *d);
	switch (in->kind) {
	case I_ZEROS: return d;
	case I_ONES:
	case I_FILL: {
		float v = in->kind == I_ONES ? 1.0f : (float)in->v[0];
		for (int i = 0; i < n; i++) d[i] = v;
		return d;
	}
	case I_RAND: {
		uint32_t s = (uint32_t)(int64_t)in->v[0];
		if (!s) s = 0x9e3779b9u;
		float scale = (float)in->v[1];
		for (int i = 0; i < n; i++) {
			float u = (float)(xorshift(&s) >> 8) / 16777216.0f;
			d[i] = (2.0f * u - 1.0f) * scale;
		}
		return d;
	}
	case I_DATA:
		if (in->nv != n) fail(f, l->file, in->line, "param '%s' needs %d values, literal has %d", pname, n, in->nv);
		for (int i = 0; i < n; i++) d[i] = (float)in->v[i];
		return d;
	case I_FILE: {
		const char *full = in->str[0] == '/' ? in->str : join(f, dir_of(f, l->file), in->str);
		size_t len = 0;
		char *raw = read_all(f, full, &len);
		if (!raw) fail(f, NULL, 0, "cannot open '%s'", full);
		if (len != (size_t)n * 4) fail(f, l->file, in->line, "'%s' has %zu bytes, param '%s' needs %d (raw little-endian f32)", full, len, pname, n * 4);
		const unsigned char *b = (const unsigned char *)raw;
		for (int i = 0; i < n; i++) {
			uint32_t w = (uint32_t)b[4 * i] | (uint32_t)b[4 * i + 1] << 8 | (uint32_t)b[4 * i + 2] << 16 | (uint32_t)b[4 * i + 3] << 24;
			memcpy(&d[i], &w, 4);
		}
		return d;
	}
	case I_ENV: {
		const char *val = getenv(in->str);
		if (!val) {
			if (in->nv < 1)
				fail(f, l->file, in->line, "environment variable %s is not set (param '%s'; give a default: env(\"%s\", 0))", in->str, pname, in->str);
			for (int i = 0; i < n; i++) d[i] = (float)in->v[0];
			return d;
		}
		const char *bad;
		int got = parse_row(val, d, n, &bad);
		if (got < 0) fail(f, l->file, in->line, "environment variable %s: bad number near '%.20s'", in->str, bad);
		if (got == 1)
			for (int i = 1; i < n; i++) d[i] = d[0];
		else if (got != n)
			fail(f, l->file, in->line, "environment variable %s has %d values, param '%s' needs %d (or 1 to fill)", in->str, got, pname, n);
		return d;
	}
	}
	return d;
}

/* ---------------------------------------------------------- liveness --- */

static void mark(F *f, const Blk *b, char *live);

static void mark_scan(F *f, const Ins *in, char *live)
{
	int any = 0;
	for (int m = 0; m < in->ny; m++)
		if (live[in->ys[m]]) live[in->y[m]] = 1, any = 1;
	for (int changed = 1; changed;) { /* a carry read by the live body is needed too */
		mark(f, in->body, live);
		changed = 0;
		for (int k = 0; k < in->nc; k++)
			if (live[in->c[k]] && !live[in->cnext[k]]) live[in->cnext[k]] = 1, changed = 1;
	}
	for (int k = 0; k < in->nc; k++)
		if (live[in->c[k]]) live[in->cinit[k]] = 1, any = 1;
	if (any)
		for (int j = 0; j < in->nx; j++) live[in->x[j]] = 1;
}

static void mark(F *f, const Blk *b, char *live)
{
	for (int i = b->len - 1; i >= 0; i--) {
		const Ins *in = &b->v[i];
		if (OPS[in->op].cls == C_SCAN) {
			mark_scan(f, in, live);
		} else if (live[in->out]) {
			if (OPS[in->op].cls == C_THINK) {
				live[in->init] = live[in->yield] = 1;
				if (in->halt >= 0) live[in->halt] = 1;
				mark(f, in->body, live);
			} else {
				for (int j = 0; j < in->na; j++) live[in->a[j]] = 1;
			}
		}
	}
}

static void sweep(F *f, Blk *b, char *live)
{
	mark(f, b, live);
	int k = 0;
	for (int i = 0; i < b->len; i++) {
		Ins *in = &b->v[i];
		if (OPS[in->op].cls == C_SCAN) {
			int nc = 0, ny = 0;
			for (int c = 0; c < in->nc; c++)
				if (live[in->c[c]]) in->c[nc] = in->c[c], in->cinit[nc] = in->cinit[c], in->cnext[nc++] = in->cnext[c];
			for (int m = 0; m < in->ny; m++)
				if (live[in->ys[m]]) in->y[ny] = in->y[m], in->ys[ny++] = in->ys[m];
			in->nc = nc;
			in->ny = ny;
			if (!nc && !ny) continue;
			in->out = nc ? in->c[0] : in->ys[0];
			sweep(f, in->body, live);
		} else {
			if (!live[in->out]) continue;
			if (OPS[in->op].cls == C_THINK) sweep(f, in->body, live);
		}
		b->v[k++] = *in;
	}
	b->len = k;
}

static void dce(F *f)
{
	char *live = fa(f, (size_t)f->nval + 1);
	live[f->output] = 1;
	for (int i = 0; i < f->nupd; i++) {
		live[f->usrc[i]] = 1;
		if (f->urows[i] >= 0) live[f->urows[i]] = 1;
	}
	sweep(f, &f->top, live);
	for (int v = 0; v < f->nval; v++)
		if (f->val[v].kind == K_PARAM && f->val[v].name && !strncmp(f->val[v].name, "__", 2) && !live[v]) f->val[v].dead = 1;
}

/* -------------------------------------------------------------- text --- */

typedef struct {
	F *f;
	char *s;
	size_t n, cap;
	int *ren;
} W;

static void put(W *w, const char *fmt, ...)
{
	va_list ap;
	for (;;) {
		va_start(ap, fmt);
		int k = vsnprintf(w->s + w->n, w->cap - w->n, fmt, ap);
		va_end(ap);
		if (k < 0) fail(w->f, NULL, 0, "formatting failed");
		if ((size_t)k < w->cap - w->n) {
			w->n += (size_t)k;
			return;
		}
		size_t cap = w->cap * 2 + (size_t)k;
		char *s = realloc(w->s, cap);
		if (!s) fail(w->f, NULL, 0, "out of memory");
		w->s = s;
		w->cap = cap;
	}
}

static void indent(W *w, int d)
{
	for (int i = 0; i < d; i++) put(w, "  ");
}

static const char *vn(W *w, int v, char *buf) /* buf holds 64 bytes */
{
	if (w->f->val[v].name) snprintf(buf, 64, "%s", w->f->val[v].name);
	else snprintf(buf, 64, "%%%d", w->ren[v]);
	return buf;
}

/* temporaries in the order a reader recreates them: pre-order, a think's
 * result before its body, a scan's carries, slices, body, then stacks */
static void number(W *w, const Blk *b, int *next)
{
	for (int i = 0; i < b->len; i++) {
		const Ins *in = &b->v[i];
		if (OPS[in->op].cls == C_SCAN) {
			for (int k = 0; k < in->nc; k++) w->ren[in->c[k]] = (*next)++;
			for (int j = 0; j < in->nx; j++) w->ren[in->xt[j]] = (*next)++;
			number(w, in->body, next);
			for (int y = 0; y < in->ny; y++) w->ren[in->ys[y]] = (*next)++;
			continue;
		}
		w->ren[in->out] = (*next)++;
		if (OPS[in->op].cls == C_THINK) number(w, in->body, next);
	}
}

static void write_block(W *w, const Blk *b, int d)
{
	F *f = w->f;
	char sh[64], n0[64], n1[64];
	for (int i = 0; i < b->len; i++) {
		const Ins *in = &b->v[i];
		indent(w, d);
		if (OPS[in->op].cls == C_SCAN) {
			put(w, "(scan %d forward\n", in->T);
			for (int k = 0; k < in->nc; k++) {
				indent(w, d + 1);
				put(w, "(carry %s %s %s)\n", vn(w, in->c[k], n0), shstr(&f->val[in->c[k]].sh, sh), vn(w, in->cinit[k], n1));
			}
			for (int j = 0; j < in->nx; j++) {
				indent(w, d + 1);
				put(w, "(in %s %s %s)\n", vn(w, in->xt[j], n0), shstr(&f->val[in->xt[j]].sh, sh), vn(w, in->x[j], n1));
			}
			indent(w, d + 1);
			put(w, "(body\n");
			write_block(w, in->body, d + 2);
			indent(w, d + 1);
			put(w, ")\n");
			for (int k = 0; k < in->nc; k++) {
				indent(w, d + 1);
				put(w, "(next %s %s)\n", vn(w, in->c[k], n0), vn(w, in->cnext[k], n1));
			}
			for (int y = 0; y < in->ny; y++) {
				indent(w, d + 1);
				put(w, "(emit %s %s %s)\n", vn(w, in->ys[y], n0), shstr(&f->val[in->ys[y]].sh, sh), vn(w, in->y[y], n1));
			}
			indent(w, d);
			put(w, ")\n");
			continue;
		}
		put(w, "(%s %s ", vn(w, in->out, n0), shstr(&f->val[in->out].sh, sh));
		switch (OPS[in->op].cls) {
		case C_CONST: put(w, "(const %.9g))\n", (double)in->k); break;
		case C_THINK:
			put(w, "(think %s %d ", vn(w, in->init, n1), in->maxit);
			if (in->eps < 0) put(w, "none\n");
			else put(w, "%.9g\n", (double)in->eps);
			write_block(w, in->body, d + 1);
			indent(w, d + 1);
			put(w, "(yield %s)", vn(w, in->yield, n1));
			if (in->halt >= 0) {
				put(w, "\n");
				indent(w, d + 1);
				put(w, "(halt %s %.9g)", vn(w, in->halt, n1), (double)in->hthr);
			}
			put(w, "))\n");
			break;
		default:
			put(w, "(%s", OPS[in->op].name);
			for (int j = 0; j < in->na; j++) put(w, " %s", vn(w, in->a[j], n1));
			put(w, "))\n");
		}
	}
}

static char *write_tgir(F *f)
{
	W w = { f, malloc(1 << 16), 0, 1 << 16, fa(f, (size_t)(f->nval + 1) * sizeof(int)) };
	if (!w.s) fail(f, NULL, 0, "out of memory");
	char sh[64], n0[64];
	int next = 0;
	for (int v = 0; v < f->nval; v++)
		if (f->val[v].kind != K_TMP && !f->val[v].dead) next++;
	number(&w, &f->top, &next);
	put(&w, "(tgir 1\n  (model %s)\n", f->name);
	for (int v = 0; v < f->nval; v++) {
		const Val *x = &f->val[v];
		if ((x->kind != K_PARAM && x->kind != K_STATE) || x->dead) continue;
		put(&w, "  (%s %s %s\n    (data", x->kind == K_STATE ? "state" : "param", x->name, shstr(&x->sh, sh));
		int k = numel(&x->sh);
		for (int i = 0; i < k; i++) {
			if (i && i % 8 == 0) put(&w, "\n         ");
			put(&w, " %.9g", (double)x->data[i]);
		}
		put(&w, "))\n");
	}
	for (int i = 0; i < f->ninputs; i++) {
		const Val *x = &f->val[f->inputs[i]];
		put(&w, "  (input %s %s)\n", x->name, shstr(&x->sh, sh));
	}
	put(&w, "  (block\n");
	write_block(&w, &f->top, 2);
	put(&w, "  )\n  (output %s)", vn(&w, f->output, n0));
	for (int i = 0; i < f->nupd; i++) {
		put(&w, "\n  (update %s %s", f->val[f->ust[i]].name, vn(&w, f->usrc[i], n0));
		if (f->urows[i] >= 0) put(&w, " %s", vn(&w, f->urows[i], n0));
		put(&w, ")");
	}
	put(&w, ")\n");
	return w.s;
}

/* ------------------------------------------------------------ driver --- */

static const char *BUILTIN[] = { "dot", "grad", "mse", "bce", "xent", "rope", "attention", "reshape", NULL };

static char *lower_module(F *f, const char *path)
{
	Prog g = { 0 };
	load_file(f, &g, path, 0, 1, NULL, 0);
	L l = { f, path, &g, { 0 }, 0, 0, NULL, NULL };
	Decl *entry = NULL;
	for (int i = 0; i < g.n; i++)
		if (g.d[i]->kind == D_MODEL) {
			if (f->name) fail(f, path, g.d[i]->line, "duplicate 'model' declaration");
			f->name = g.d[i]->name;
		}
	if (!f->name) fail(f, path, 1, "missing 'model <name>' declaration");
	int ndefs = 0;
	for (int i = 0; i < g.n; i++) {
		Decl *d = g.d[i];
		if (d->kind == D_PARAM || d->kind == D_STATE) {
			if (env_get(&l.globals, d->name) >= 0) fail(f, path, d->line, "duplicate param or state '%s'", d->name);
			int v = newval(f, d->kind == D_STATE ? K_STATE : K_PARAM, &d->sh, d->name);
			f->val[v].data = materialize(&l, &d->init, &d->sh, d->name);
			env_set(f, &l.globals, d->name, v);
		} else if (d->kind == D_DEF) {
			for (int j = 0; j < i; j++)
				if (g.d[j]->kind == D_DEF && !strcmp(g.d[j]->name, d->name)) fail(f, path, d->line, "duplicate def '%s'", d->name);
			int shadow = op_of(d->name) >= 0;
			for (int k = 0; BUILTIN[k]; k++) shadow |= !strcmp(d->name, BUILTIN[k]);
			if (shadow) fail(f, path, d->line, "'%s' shadows a builtin", d->name);
			if (!strcmp(d->name, "forward")) entry = d;
			ndefs++;
		}
	}
	for (int i = 0; i < g.n; i++)
		if (g.d[i]->kind == D_DEF)
			for (int j = 0; j < g.d[i]->nargs; j++)
				if (env_get(&l.globals, g.d[i]->an[j]) >= 0)
					fail(f, path, g.d[i]->line, "argument '%s' shadows a param", g.d[i]->an[j]);
	if (!entry) fail(f, path, 1, "missing entry point 'def forward(...)'");
	if (entry->nargs == 0) fail(f, path, entry->line, "'forward' needs at least one input");
	Env e = { 0 };
	for (int i = 0; i < entry->nargs; i++) {
		if (env_get(&e, entry->an[i]) >= 0) fail(f, path, entry->line, "duplicate input '%s'", entry->an[i]);
		env_set(f, &e, entry->an[i], newval(f, K_INPUT, &entry->as[i], entry->an[i]));
	}
	int r = lower_block(&l, &f->top, &e, entry->body, entry->nbody, 1, entry->bline);
	if (!sheq(&entry->sh, &f->val[r].sh)) fail(f, path, entry->line, "'forward' return shape does not match its declaration");
	f->output = r;
	dce(f);
	return write_tgir(f);
}

char *tgf_lower(const char *path, char *err, size_t errn)
{
	F *f = calloc(1, sizeof *f);
	if (!f) {
		snprintf(err, errn, "out of memory");
		return NULL;
	}
	f->err = err;
	f->errn = errn;
	err[0] = 0;
	char *out = NULL;
	if (!setjmp(f->jb)) out = lower_module(f, path);
	for (int i = 0; i < f->mem.n; i++) free(f->mem.p[i]);
	free(f->mem.p);
	free(f);
	return out;
}
