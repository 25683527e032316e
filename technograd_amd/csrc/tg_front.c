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
#include <limits.h>
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
	int64_t n = 1; /* element counts are ints everywhere below: larger tensors are refused here */
	for (int i = 0; i < sh->rank; i++)
		if ((n *= sh->dim[i] > 0 ? sh->dim[i] : 1) > INT_MAX) {
			snprintf(f->err, f->errn, "a tensor of more than %d elements", INT_MAX);
			longjmp(f->jb, 1);
		}
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

/* the token at the cursor; take() also moves past it (never past the end) */
static Tok *look(P *p) { return &p->t[p->i]; }
static Tok *take(P *p)
{
	Tok *t = &p->t[p->i];
	if (t->k != T_EOF) p->i++;
	return t;
}

/* how a diagnostic names a token */
static const char *tokname(Tok *t)
{
	switch (t->k) {
	case T_NL: return "end of line";
	case T_INDENT: return "indent";
	case T_DEDENT: return "dedent";
	case T_EOF: return "end of file";
	default: return t->s;
	}
}

static int at_punct(Tok *t, const char *s) { return t->k == T_OP && !strcmp(t->s, s); }
static int at_word(Tok *t, const char *s) { return t->k == T_NAME && !strcmp(t->s, s); }

static void need_punct(P *p, const char *s)
{
	Tok *t = take(p);
	if (!at_punct(t, s)) fail(p->f, p->file, t->line, "expected '%s', got '%s'", s, tokname(t));
}

static Tok *need_kind(P *p, int k, const char *what)
{
	Tok *t = take(p);
	if (t->k != k) fail(p->f, p->file, t->line, "expected %s, got '%s'", what, tokname(t));
	return t;
}

static Tok *need_ident(P *p)
{
	Tok *t = need_kind(p, T_NAME, "name");
	for (int i = 0; KW[i]; i++)
		if (!strcmp(t->s, KW[i])) fail(p->f, p->file, t->line, "'%s' is a reserved word", t->s);
	return t;
}

static double signed_lit(P *p)
{
	int neg = 0;
	if (at_punct(look(p), "-")) take(p), neg = 1;
	Tok *t = need_kind(p, T_NUM, "number");
	return neg ? -t->n : t->n;
}

/* v is a whole number in [1, max] (compared as a double, so no value outside int is converted) */
static int whole_in(double v, double max) { return v >= 1 && v <= max && v == floor(v); }

static int count_lit(P *p)
{
	Tok *t = need_kind(p, T_NUM, "integer");
	if (!whole_in(t->n, 1 << 24)) fail(p->f, p->file, t->line, "expected positive integer, got '%s'", t->s);
	return (int)t->n;
}

static Sh type(P *p)
{
	Tok *t = take(p);
	if (!at_word(t, "f32")) fail(p->f, p->file, t->line, "expected type 'f32', got '%s'", tokname(t));
	Sh s = { 0, { 0 } };
	if (at_punct(look(p), "[")) {
		take(p);
		for (;;) {
			if (s.rank >= MAXRANK) fail(p->f, p->file, t->line, "rank exceeds %d", MAXRANK);
			s.dim[s.rank++] = count_lit(p);
			if (at_punct(look(p), "]")) {
				take(p);
				break;
			}
			need_punct(p, ",");
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
	if (at_punct(look(p), "[")) {
		take(p);
		for (;;) {
			literal(p, in);
			if (at_punct(look(p), "]")) {
				take(p);
				return;
			}
			need_punct(p, ",");
		}
	}
	init_add(p, in, signed_lit(p));
}

static Init initializer(P *p)
{
	Tok *t = look(p);
	Init in = { I_DATA, 0, t->line, 0, NULL, NULL };
	if (at_word(t, "zeros") || at_word(t, "ones")) {
		take(p);
		in.kind = at_word(t, "zeros") ? I_ZEROS : I_ONES;
	} else if (at_word(t, "fill")) {
		take(p);
		need_punct(p, "(");
		in.kind = I_FILL;
		init_add(p, &in, signed_lit(p));
		need_punct(p, ")");
	} else if (at_word(t, "rand")) {
		take(p);
		need_punct(p, "(");
		in.kind = I_RAND;
		init_add(p, &in, signed_lit(p));
		need_punct(p, ",");
		init_add(p, &in, signed_lit(p));
		need_punct(p, ")");
	} else if (at_word(t, "file")) {
		take(p);
		need_punct(p, "(");
		in.kind = I_FILE;
		in.str = need_kind(p, T_STR, "string")->s;
		need_punct(p, ")");
	} else if (at_word(t, "env")) {
		take(p);
		need_punct(p, "(");
		in.kind = I_ENV;
		in.str = need_kind(p, T_STR, "string")->s;
		if (at_punct(look(p), ",")) take(p), init_add(p, &in, signed_lit(p));
		need_punct(p, ")");
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
	Tok *t = take(p);
	if (t->k == T_NUM) {
		Ex *e = ex_new(p, E_NUM, t->line);
		e->num = t->n;
		return e;
	}
	if (at_punct(t, "(")) {
		Ex *e = expr(p);
		need_punct(p, ")");
		return e;
	}
	if (t->k == T_NAME) {
		for (int i = 0; KW[i]; i++)
			if (!strcmp(t->s, KW[i])) fail(p->f, p->file, t->line, "unexpected keyword '%s' in expression", t->s);
		if (at_punct(look(p), "(")) {
			take(p);
			Ex *c = ex_new(p, E_CALL, t->line);
			c->name = t->s;
			if (at_punct(look(p), ")")) {
				take(p);
				return c;
			}
			for (;;) {
				ex_arg(p, c, expr(p));
				if (at_punct(look(p), ")")) {
					take(p);
					return c;
				}
				need_punct(p, ",");
			}
		}
		Ex *e = ex_new(p, E_REF, t->line);
		e->name = t->s;
		return e;
	}
	fail(p->f, p->file, t->line, "expected expression, got '%s'", tokname(t));
	return NULL;
}

static Ex *unary(P *p)
{
	if (at_punct(look(p), "-")) {
		int line = take(p)->line;
		Tok *t = look(p);
		if (t->k == T_NUM) { /* a negative literal is one number */
			take(p);
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
		Tok *t = look(p);
		const char *op = at_punct(t, "*") ? "mul" : at_punct(t, "/") ? "div" : at_punct(t, "@") ? "matmul" : NULL;
		if (!op) return e;
		take(p);
		e = call(p, op, e, unary(p), t->line);
	}
}

static Ex *expr(P *p)
{
	Ex *e = term(p);
	for (;;) {
		Tok *t = look(p);
		const char *op = at_punct(t, "+") ? "add" : at_punct(t, "-") ? "sub" : NULL;
		if (!op) return e;
		take(p);
		e = call(p, op, e, term(p), t->line);
	}
}

static void block(P *p, St ***body, int *n, int *bline);

static const char **name_push(P *p, const char **a, int n, const char *s)
{
	const char **r = fa(p->f, (size_t)(n + 1) * sizeof *r);
	if (n) memcpy(r, a, (size_t)n * sizeof *r);
	r[n] = s;
	return r;
}

/* Statements. Each form after its leading word has a handler (the word is
 * consumed); a line that starts with none of them is an assignment. The
 * token sequence each form accepts, and the diagnostic for the first token
 * that breaks it, are the surface grammar's (src/parse.c); the pieces shared
 * by several forms are the helpers below. */

static void line_end(P *p) { need_kind(p, T_NL, "end of line"); }

static Ex *assigned(P *p) /* "= expr" */
{
	need_punct(p, "=");
	return expr(p);
}

/* item, then more items while a comma follows */
static void comma_list(P *p, void (*item)(P *p, St *s), St *s)
{
	for (item(p, s); at_punct(look(p), ","); item(p, s)) take(p);
}

/* the word w or fail with msg (a format with the got-token last) */
static Tok *need_word(P *p, const char *w, const char *msg, const char *arg)
{
	Tok *t = take(p);
	if (!at_word(t, w)) {
		if (arg) fail(p->f, p->file, t->line, msg, arg, tokname(t));
		fail(p->f, p->file, t->line, msg, tokname(t));
	}
	return t;
}

static St *st_return(P *p, St *s)
{
	s->kind = S_RETURN;
	s->e = expr(p);
	line_end(p);
	return s;
}

static void opt_item(P *p, St *s)
{
	(void)s;
	need_kind(p, T_NAME, "option name");
	need_punct(p, "=");
	signed_lit(p);
}

static void over_item(P *p, St *s)
{
	(void)s;
	need_ident(p);
}

static St *st_train(P *p, St *s) /* parsed for its diagnostics; lowering refuses it */
{
	s->kind = S_TRAIN;
	s->e = expr(p);
	if (at_word(look(p), "with")) {
		take(p);
		need_kind(p, T_NAME, "optimizer name");
		if (at_punct(look(p), "(")) {
			take(p);
			for (opt_item(p, s); !at_punct(look(p), ")"); opt_item(p, s)) need_punct(p, ",");
			take(p);
		}
	}
	if (at_word(look(p), "over")) {
		take(p);
		comma_list(p, over_item, s);
	}
	line_end(p);
	return s;
}

static St *st_update(P *p, St *s)
{
	s->kind = S_UPDATE;
	s->name = need_ident(p)->s;
	if (at_punct(look(p), "[")) {
		take(p);
		s->rows = expr(p);
		need_punct(p, "]");
	}
	s->e = assigned(p);
	line_end(p);
	return s;
}

static void carry_item(P *p, St *s)
{
	s->cs = name_push(p, s->cs, s->ncs++, need_ident(p)->s);
}

static void slice_item(P *p, St *s)
{
	Tok *n = need_ident(p);
	need_word(p, "in", "expected 'in' after scan slice '%s', got '%s'", n->s);
	Ex *e = expr(p);
	Ex **xe = fa(p->f, (size_t)(s->nx + 1) * sizeof *xe);
	if (s->nx) memcpy(xe, s->xe, (size_t)s->nx * sizeof *xe);
	xe[s->nx] = e;
	s->xe = xe;
	s->xn = name_push(p, s->xn, s->nx++, n->s);
}

static St *st_scan(P *p, St *s)
{
	s->kind = S_SCAN;
	comma_list(p, carry_item, s);
	need_word(p, "over", "expected 'over' after the scan carries, got '%s'", NULL);
	comma_list(p, slice_item, s);
	need_punct(p, ":");
	block(p, &s->body, &s->nbody, &s->bline);
	return s;
}

static St *st_emit(P *p, St *s)
{
	s->kind = S_EMIT;
	s->name = need_ident(p)->s;
	s->e = assigned(p);
	line_end(p);
	return s;
}

/* think STATE for N [until EPS | halt NAME [at THRESHOLD]]: BLOCK */
static St *st_think(P *p, St *s)
{
	s->kind = S_THINK;
	s->name = need_ident(p)->s;
	need_word(p, "for", "expected 'for' after think state, got '%s'", NULL);
	s->maxit = count_lit(p);
	s->eps = -1;
	Tok *t = look(p);
	if (at_word(t, "until")) {
		take(p);
		s->eps = signed_lit(p);
		if (s->eps < 0) fail(p->f, p->file, s->line, "halting threshold must be >= 0");
	} else if (at_word(t, "halt")) {
		take(p);
		s->has_halt = 1;
		s->halt = need_ident(p)->s;
		s->hthr = 0.5;
		if (at_word(look(p), "at")) {
			take(p);
			s->hthr = signed_lit(p);
			if (s->hthr <= 0 || s->hthr >= 1) fail(p->f, p->file, s->line, "halting threshold must be in (0, 1)");
		}
	}
	need_punct(p, ":");
	block(p, &s->body, &s->nbody, &s->bline);
	return s;
}

static const struct {
	const char *word;
	St *(*form)(P *p, St *s);
} STMT_FORMS[] = {
	{ "return", st_return }, { "train", st_train }, { "update", st_update },
	{ "scan", st_scan },     { "emit", st_emit },   { "think", st_think },
};

static St *stmt(P *p)
{
	Tok *t = look(p);
	St *s = fa(p->f, sizeof *s);
	s->line = t->line;
	for (size_t i = 0; i < sizeof STMT_FORMS / sizeof STMT_FORMS[0]; i++)
		if (at_word(t, STMT_FORMS[i].word)) {
			take(p);
			return STMT_FORMS[i].form(p, s);
		}
	s->kind = S_SET; /* NAME = expr */
	s->name = need_ident(p)->s;
	s->e = assigned(p);
	line_end(p);
	return s;
}

/* NL INDENT statement... DEDENT */
static void block(P *p, St ***body, int *n, int *bline)
{
	line_end(p);
	*bline = need_kind(p, T_INDENT, "indented block")->line;
	St **v = NULL;
	int len = 0;
	while (look(p)->k != T_DEDENT && look(p)->k != T_EOF) {
		St *s = stmt(p);
		St **grown = fa(p->f, (size_t)(len + 1) * sizeof *grown);
		if (len) memcpy(grown, v, (size_t)len * sizeof *grown);
		grown[len++] = s;
		v = grown;
	}
	need_kind(p, T_DEDENT, "dedent");
	*body = v;
	*n = len;
}

static Decl *decl(P *p)
{
	Tok *t = take(p);
	Decl *d = fa(p->f, sizeof *d);
	d->line = t->line;
	if (at_word(t, "import")) {
		d->kind = D_IMPORT;
		d->str = need_kind(p, T_STR, "import path string")->s;
		need_kind(p, T_NL, "end of line");
	} else if (at_word(t, "model")) {
		d->kind = D_MODEL;
		d->name = need_ident(p)->s;
		need_kind(p, T_NL, "end of line");
	} else if (at_word(t, "param") || at_word(t, "state")) {
		d->kind = at_word(t, "param") ? D_PARAM : D_STATE;
		d->name = need_ident(p)->s;
		need_punct(p, ":");
		d->sh = type(p);
		need_punct(p, "=");
		d->init = initializer(p);
		need_kind(p, T_NL, "end of line");
	} else if (at_word(t, "def")) {
		d->kind = D_DEF;
		d->name = need_ident(p)->s;
		need_punct(p, "(");
		if (!at_punct(look(p), ")")) {
			for (;;) {
				Tok *a = need_ident(p);
				need_punct(p, ":");
				Sh sh = type(p);
				Sh *as = fa(p->f, (size_t)(d->nargs + 1) * sizeof *as);
				if (d->nargs) memcpy(as, d->as, (size_t)d->nargs * sizeof *as);
				as[d->nargs] = sh;
				d->as = as;
				d->an = name_push(p, d->an, d->nargs++, a->s);
				if (at_punct(look(p), ")")) break;
				need_punct(p, ",");
			}
		}
		need_punct(p, ")");
		need_punct(p, "->");
		d->sh = type(p);
		need_punct(p, ":");
		block(p, &d->body, &d->nbody, &d->bline);
	} else {
		fail(p->f, p->file, d->line, "expected 'import', 'model', 'param', 'state' or 'def', got '%s'", tokname(t));
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
		Tok *t = look(&p);
		if (t->k == T_EOF) break;
		if (t->k == T_NL) {
			take(&p);
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

/* ---- builtin expansions ----
 * The builtins the reference expands into table operations (the losses,
 * rope, attention, take_along) are written here as expression trees over the
 * call's values, one tree per intermediate the reference names. tree_emit()
 * creates a tree's instructions in the order the reference's build creates
 * them: its builder calls take their operands as nested calls, which that
 * build evaluates last operand first, so a tree is emitted in post-order
 * with the operands visited from the last to the first. The trees live in
 * compound literals of the enclosing block. */
typedef struct Tn {
	char kind;              /* 'v' a value, 'k' a scalar constant, 'o' an operation, 'r' a reshape */
	int v;                  /* 'v' */
	float k;                /* 'k' */
	const char *op;         /* 'o' */
	const struct Tn *a, *b; /* operands ('o': b NULL when unary; 'r': a) */
	const Sh *to;           /* 'r' */
} Tn;
#define TV(x) (&(Tn){ 'v', (x), 0, NULL, NULL, NULL, NULL })
#define TK(x) (&(Tn){ 'k', -1, (float)(x), NULL, NULL, NULL, NULL })
#define T1(o, x) (&(Tn){ 'o', -1, 0, (o), (x), NULL, NULL })
#define T2(o, x, y) (&(Tn){ 'o', -1, 0, (o), (x), (y), NULL })
#define TR(x, s) (&(Tn){ 'r', -1, 0, NULL, (x), NULL, (s) })

static int tree_emit(L *l, Blk *b, const Tn *t, int line)
{
	switch (t->kind) {
	case 'v': return t->v;
	case 'k': return konst(l, b, t->k);
	case 'r': return reshape_to(l, b, tree_emit(l, b, t->a, line), t->to);
	default: {
		const int q = t->b ? tree_emit(l, b, t->b, line) : -1; /* the last operand first */
		const int r = tree_emit(l, b, t->a, line);
		return op2(l, b, t->op, r, q, line);
	}
	}
}

/* mse, bce, xent of prediction p and target t (shapes checked by the caller) */
static int lower_loss(L *l, Blk *b, const char *fn, int p, int t, int line)
{
	F *f = l->f;
	if (!strcmp(fn, "mse")) { /* mean((p - t)^2) */
		const int d = tree_emit(l, b, T2("sub", TV(p), TV(t)), line);
		return tree_emit(l, b, T1("mean", T2("mul", TV(d), TV(d))), line);
	}
	if (!strcmp(fn, "bce")) { /* -mean(t log(p + 1e-7) + (1 - t) log(1 - p + 1e-7)) */
		const int lp = tree_emit(l, b, T1("log", T2("add", TV(p), TK(1e-7f))), line);
		const int lq = tree_emit(l, b, T1("log", T2("add", T2("sub", TK(1), TV(p)), TK(1e-7f))), line);
		const int sm = tree_emit(l, b, T2("add", T2("mul", TV(t), TV(lp)), T2("mul", T2("sub", TK(1), TV(t)), TV(lq))), line);
		return tree_emit(l, b, T1("neg", T1("mean", TV(sm))), line);
	}
	const int rk = f->val[p].sh.rank; /* xent: -sum(t log(softmax(p) + 1e-12)), averaged over a batch's rows */
	if (rk != 1 && rk != 2) fail(f, l->file, line, "'xent' needs logits of shape (C) or a batch (B, C), with one-hot targets");
	const int ls = tree_emit(l, b, T1("log", T2("add", T1("softmax", TV(p)), TK(1e-12f))), line);
	int sm = tree_emit(l, b, T1("sum", T2("mul", TV(t), TV(ls))), line);
	if (rk == 2) sm = tree_emit(l, b, T2("div", TV(sm), TK((float)f->val[p].sh.dim[0])), line);
	return tree_emit(l, b, T1("neg", TV(sm)), line);
}

/* rope(x, position): x cos(a) + (x @ swap) sin(a), a = freq * position */
static int lower_rope(L *l, Blk *b, Env *e, Ex *x)
{
	F *f = l->f;
	const int line = x->line;
	if (x->nargs != 2) fail(f, l->file, line, "'rope' takes (x, position)");
	const int v = lower_expr(l, b, e, x->args[0]), pos = lower_expr(l, b, e, x->args[1]);
	const Sh xs = f->val[v].sh, ps = f->val[pos].sh;
	const int d = xs.dim[xs.rank - 1];
	const int shapes = (xs.rank == 1 && ps.rank == 0) || (xs.rank == 2 && ps.rank == 1 && ps.dim[0] == xs.dim[0]);
	if (!shapes || d % 2) fail(f, l->file, line, "'rope' takes x (d) with a scalar position or x (T, d) with positions (T), d even");
	if ((int64_t)d * d > INT_MAX) fail(f, l->file, line, "'rope' dimension %d too large (its swap matrix has d x d entries)", d);
	/* frequencies 10000^(-2 floor(i / 2) / d); swap maps each pair (x0, x1) to (-x1, x0) under x @ swap */
	float *freq = fa(f, (size_t)d * sizeof *freq), *swap = fa(f, (size_t)d * (size_t)d * sizeof *swap);
	for (int i = 0; i < d; i++) freq[i] = (float)pow(10000.0, -(double)(i / 2 * 2) / d);
	for (int pr = 0; pr < d / 2; pr++) swap[(2 * pr) * d + 2 * pr + 1] = 1, swap[(2 * pr + 1) * d + 2 * pr] = -1;
	char name[64];
	const Sh s1 = { 1, { d } }, s2 = { 2, { d, d } };
	snprintf(name, sizeof name, "__rope_freq_%d", d);
	const int fv = const_param(l, name, &s1, freq);
	snprintf(name, sizeof name, "__swap_%d", d);
	const int sv = const_param(l, name, &s2, swap);
	const int ang = tree_emit(l, b, xs.rank == 1 ? T2("mul", TV(fv), TV(pos)) : T2("outer", TV(pos), TV(fv)), line);
	return tree_emit(l, b, T2("add", T2("mul", TV(v), T1("cos", TV(ang))), T2("mul", T2("matmul", TV(v), TV(sv)), T1("sin", TV(ang)))), line);
}

/* attention(Q, K, V, window): softmax(Q K^T / sqrt(d) + causal window mask) V */
static int lower_attention(L *l, Blk *b, Env *e, Ex *x)
{
	F *f = l->f;
	const int line = x->line;
	if (x->nargs != 4) fail(f, l->file, line, "'attention' takes (Q, K, V, window)");
	const Ex *wd = x->args[3];
	if (!is_num(wd) || !whole_in(wd->num, INT_MAX)) fail(f, l->file, line, "'attention' window must be a positive integer literal");
	const int win = (int)wd->num;
	const int q = lower_expr(l, b, e, x->args[0]), k = lower_expr(l, b, e, x->args[1]), v = lower_expr(l, b, e, x->args[2]);
	const Sh qs = f->val[q].sh, ks = f->val[k].sh, vs = f->val[v].sh;
	if (qs.rank != 2 || !sheq(&qs, &ks) || vs.rank != 2 || vs.dim[0] != qs.dim[0])
		fail(f, l->file, line, "'attention' needs Q and K of one shape (T, d) and V (T, e)");
	const int T = qs.dim[0];
	float *mask = fa(f, (size_t)T * (size_t)T * sizeof *mask); /* 0 where query t sees key s: s <= t, t - s < window */
	for (int t = 0; t < T; t++)
		for (int sk = 0; sk < T; sk++) mask[t * T + sk] = sk <= t && t - sk < win ? 0.0f : -1e9f;
	char name[64];
	const Sh ms = { 2, { T, T } };
	snprintf(name, sizeof name, "__causal_%d_%d", T, win);
	const int mv = const_param(l, name, &ms, mask);
	const float inv = (float)(1.0 / sqrt((double)qs.dim[1]));
	const int sc = tree_emit(l, b, T2("add", T2("mul", T2("matmul", TV(q), T1("transpose", TV(k))), TK(inv)), TV(mv)), line);
	return tree_emit(l, b, T2("matmul", T1("softmax", TV(sc)), TV(v)), line);
}

/* take_along(x, i): the gather along the last axis as one take over the
 * flattened rows; an index outside [0, n) reads element -1 of the flattened
 * x's row... taken as zero by the in-range mask (i + 1) and (n - i) steps */
static int lower_take_along(L *l, Blk *b, Env *e, Ex *x)
{
	F *f = l->f;
	const int line = x->line;
	char s0[64], s1[64];
	if (x->nargs != 2) fail(f, l->file, line, "'take_along' takes (x, indices)");
	const int v = lower_expr(l, b, e, x->args[0]), iv = lower_expr(l, b, e, x->args[1]);
	const Sh xs = f->val[v].sh, is = f->val[iv].sh;
	int same = xs.rank >= 1 && is.rank == xs.rank;
	for (int d = 0; same && d < xs.rank - 1; d++) same = xs.dim[d] == is.dim[d];
	if (!same)
		fail(f, l->file, line, "'take_along' needs x (..., n) and indices (..., k) with the same leading dimensions; got %s and %s",
		     shstr(&xs, s0), shstr(&is, s1));
	const int n = xs.dim[xs.rank - 1], k = is.dim[is.rank - 1], R = numel(&xs) / n;
	int inr = tree_emit(l, b, T2("mul", T1("step", T2("add", TV(iv), TK(1))), T1("step", T2("sub", TK(n), TV(iv)))), line);
	int at = iv;
	const Sh rk = { 2, { R, k } };
	if (R > 1) { /* row r's indices offset by r n, over the flattened rows */
		float *off = fa(f, (size_t)R * sizeof *off);
		for (int r = 0; r < R; r++) off[r] = (float)r * (float)n;
		char name[64];
		const Sh os = { 2, { R, 1 } };
		snprintf(name, sizeof name, "__rowoff_%d_%d", R, n);
		const int ov = const_param(l, name, &os, off);
		at = tree_emit(l, b, T2("add", TR(TV(iv), &rk), TV(ov)), line);
		inr = tree_emit(l, b, TR(TV(inr), &rk), line);
	}
	const int idx = tree_emit(l, b, T2("sub", T2("add", T2("mul", TV(at), TV(inr)), TV(inr)), TK(1)), line);
	const Sh flat = { 2, { R * n, 1 } }, list = { 1, { R * k } };
	const int g = tree_emit(l, b, T2("take", TR(TV(v), &flat), TR(TV(idx), &list)), line);
	return tree_emit(l, b, TR(TV(g), &is), line);
}

static int lower_expr(L *l, Blk *b, Env *e, Ex *x)
{
	F *f = l->f;
	char s0[64], s1[64];
	if (x->kind == E_NUM) return konst(l, b, (float)x->num);
	if (x->kind == E_REF) return lookup(l, e, x->name, x->line);
	const char *fn = x->name;
	if (!strcmp(fn, "grad")) fail(f, l->file, x->line, "'grad' (automatic differentiation) is not part of the batch backend's front end");
	if (!strcmp(fn, "rope")) return lower_rope(l, b, e, x);
	if (!strcmp(fn, "attention")) return lower_attention(l, b, e, x);
	if (!strcmp(fn, "topk") || !strcmp(fn, "memory_scan") || !strcmp(fn, "memory_final") || !strcmp(fn, "suffix_match"))
		fail(f, l->file, x->line, "'%s' is not run by the batch backend", fn);
	if (!strcmp(fn, "take_along")) return lower_take_along(l, b, e, x);
	if (!strcmp(fn, "reshape")) {
		Sh to = { 0, { 0 } };
		if (x->nargs < 2 || x->nargs - 1 > MAXRANK) fail(f, l->file, x->line, "'reshape' takes a tensor and 1 to %d dimensions", MAXRANK);
		for (int i = 1; i < x->nargs; i++) {
			Ex *d = x->args[i];
			if (!is_num(d) || !whole_in(d->num, INT_MAX))
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
		return lower_loss(l, b, fn, args[0], args[1], x->line);
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
		/* the seed's low 32 bits as an int64; outside int64 (and NaN) the x86-64
		 * conversion the reference's build uses gives INT64_MIN, low bits 0 */
		const double sv = in->v[0];
		uint32_t s = sv >= -9223372036854775808.0 && sv < 9223372036854775808.0 ? (uint32_t)(int64_t)sv : 0u;
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

/* What is kept: every value the output or a state update needs, closed
 * under "is computed from". Each value has at most one definition: an
 * instruction's output, a think loop's state (needing its init, its yield
 * and its halting value), or a scan's carry or stack; a needed carry needs
 * its initial and next values, a needed stack its stacked body value, and
 * either needs all of the scan's sliced inputs. Params, states, inputs and
 * a loop's per-step slices have no definition here. Instructions are pure:
 * one whose value is not needed is dropped, a scan keeps its needed carries
 * and stacks (its result becomes the first of them) and goes when none is
 * left. */

enum { DEF_NONE, DEF_INS, DEF_CARRY, DEF_STACK };

typedef struct {
	char kind;
	int idx;        /* DEF_CARRY / DEF_STACK: which carry or stack */
	const Ins *ins; /* the defining instruction */
} Def;

static void index_defs(const Blk *b, Def *def)
{
	for (int i = 0; i < b->len; i++) {
		const Ins *in = &b->v[i];
		if (OPS[in->op].cls == C_SCAN) {
			for (int k = 0; k < in->nc; k++) def[in->c[k]] = (Def){ DEF_CARRY, k, in };
			for (int m = 0; m < in->ny; m++) def[in->ys[m]] = (Def){ DEF_STACK, m, in };
			index_defs(in->body, def);
			continue;
		}
		def[in->out] = (Def){ DEF_INS, 0, in };
		if (OPS[in->op].cls == C_THINK) index_defs(in->body, def);
	}
}

typedef struct {
	char *live;
	int *todo, n;
} Need;

static void need(Need *w, int v)
{
	if (v < 0 || w->live[v]) return;
	w->live[v] = 1;
	w->todo[w->n++] = v;
}

static void close_needs(Need *w, const Def *def)
{
	while (w->n) {
		const int v = w->todo[--w->n];
		const Def *d = &def[v];
		const Ins *in = d->ins;
		if (d->kind == DEF_NONE) continue;
		if (d->kind == DEF_INS) {
			if (OPS[in->op].cls == C_THINK) {
				need(w, in->init);
				need(w, in->yield);
				need(w, in->halt);
			} else {
				for (int j = 0; j < in->na; j++) need(w, in->a[j]);
			}
			continue;
		}
		if (d->kind == DEF_CARRY) need(w, in->cinit[d->idx]), need(w, in->cnext[d->idx]);
		else need(w, in->y[d->idx]);
		for (int j = 0; j < in->nx; j++) need(w, in->x[j]);
	}
}

/* drops what is not needed from b, in place, keeping the order of the rest */
static void drop_unneeded(Blk *b, const char *live)
{
	int kept = 0;
	for (int i = 0; i < b->len; i++) {
		Ins in = b->v[i];
		if (OPS[in.op].cls == C_SCAN) {
			int nc = 0, ny = 0;
			for (int k = 0; k < in.nc; k++)
				if (live[in.c[k]]) in.c[nc] = in.c[k], in.cinit[nc] = in.cinit[k], in.cnext[nc] = in.cnext[k], nc++;
			for (int m = 0; m < in.ny; m++)
				if (live[in.ys[m]]) in.y[ny] = in.y[m], in.ys[ny] = in.ys[m], ny++;
			if (!nc && !ny) continue;
			in.nc = nc, in.ny = ny;
			in.out = nc ? in.c[0] : in.ys[0];
			drop_unneeded(in.body, live);
		} else {
			if (!live[in.out]) continue;
			if (OPS[in.op].cls == C_THINK) drop_unneeded(in.body, live);
		}
		b->v[kept++] = in;
	}
	b->len = kept;
}

static void dce(F *f)
{
	Def *def = fa(f, (size_t)(f->nval + 1) * sizeof *def);
	Need w = { fa(f, (size_t)f->nval + 1), fa(f, (size_t)(f->nval + 1) * sizeof(int)), 0 };
	index_defs(&f->top, def);
	need(&w, f->output);
	for (int i = 0; i < f->nupd; i++) need(&w, f->usrc[i]), need(&w, f->urows[i]);
	close_needs(&w, def);
	drop_unneeded(&f->top, w.live);
	for (int v = 0; v < f->nval; v++) /* generated constants nothing reads any more are not written */
		if (f->val[v].kind == K_PARAM && f->val[v].name && !strncmp(f->val[v].name, "__", 2) && !w.live[v]) f->val[v].dead = 1;
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
