/* TEST INFRASTRUCTURE ONLY — oracle Q16.16 interpreter.
 *
 * Restates the fixed-point runtime (runtime/tg_rtq.h) and the way a
 * `tgc c --fixed` unit calls it (src/cgen.c:100-314): one kernel per
 * instruction over int32 Q16.16 values, 64-bit accumulation rounded once,
 * saturation instead of wrap-around, params converted with to_fixed(v, 16)
 * (cgen.c:76-82, :449-455), quantized scales in Q7.24 (cgen.c:442), think
 * thresholds as to_fixed(eps, 16) with a positive eps never rounding to zero
 * (cgen.c:286-290), learned halting in Q16.16 (cgen.c:295-305).
 *
 * Function map (reference -> here): tg_sat/tg_fmul/tg_fdiv/tg_absq
 * (tg_rtq.h:30-38) -> sat/fmul/fdiv/absq; tg_expq (:61-74) -> expq; tg_logq
 * (:77-90) -> logq; tg_isqrt64 (:92-102) -> isqrt64; tg_sinq (:105-119) ->
 * sinq; tg_tanhq/tg_sigmoidq (:132-144); unary kernels (:121-158); tg_matmul
 * (:162-170); tg_qscale/tg_matmul_qa/qb (:183-201); tg_softmax/tg_rmsnorm
 * (:203-225); tg_sum/tg_mean/tg_transpose/tg_outer/tg_delta (:226-243);
 * tg_ell_idx (:246-250) for take.
 *
 * Constants are derived from their definitions, not tabulated: the exp
 * polynomial uses round(2^30 / j!) for j = 0..8; ln 2, pi, pi/2, 2 pi and the
 * gelu coefficients are round(value * 2^16); 1e-6 in Q32 is round(1e-6 * 2^32).
 *
 * Pinned by: the tests/golden fixtures that carry Q16.16 data (outputs and
 * steps of the reference's own emitted `tgc c --fixed` unit: src/cgen.c
 * compiled from /root/reference by oracle/Makefile into oracle/_ref, the unit
 * compiled with cc, over all 256 inputs of latent_reasoner's {0,1}^8 domain
 * and random inputs: byte-identical outputs and steps; a test also runs the
 * unit on 8448 fresh rows of config 4's model), closed forms in tests/ (isqrt64 against
 * integer square roots, fdiv against exact rational rounding, expq against
 * exp within its polynomial error), and the reference's fixed-vs-float bound
 * (tests/run.sh:306-322: max |fixed - float| < 5e-4). */
#include "tgo.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define ONE 65536
#define MAXV 2147483647
#define MINV (-2147483647 - 1)


/* Test-only: a planted mistake in the think loop's halting test, so a test can
 * show that comparing with the reference's emitted unit catches it
 * (0 = none, 1 = `d < thr` for `d <= thr`, 2 = threshold one below). */
int tgo_plant;

static int32_t sat(int64_t v) { return v > MAXV ? MAXV : v < MINV ? MINV : (int32_t)v; }
static int64_t asr(int64_t v, int s) { return v >> s; } /* arithmetic, as gcc and clang implement >> on int64 */
static int32_t fmul(int32_t a, int32_t b) { return sat(asr((int64_t)a * b + 32768, 16)); }
static int32_t fdiv(int32_t a, int32_t b)
{
	if (b == 0) return a > 0 ? MAXV : a < 0 ? MINV : 0;
	int64_t n = (int64_t)a * 65536, h = b > 0 ? b / 2 : -(b / 2);
	return sat(((n >= 0) == (b > 0) ? n + h : n - h) / b);
}
static int32_t absq(int32_t a) { return a < 0 ? (a == MINV ? MAXV : -a) : a; }

static int64_t EXPC[9];
static int64_t LN2_Q16, PI_Q16, TWO_PI_Q16, HALF_PI_Q16, GELU_A, GELU_B, EPS_Q32, EXP_HI;

static void init_consts(void)
{
	if (EXPC[0]) return;
	int64_t f = 1;
	for (int j = 0; j <= 8; j++) {
		if (j) f *= j;
		EXPC[j] = (((int64_t)1 << 30) + f / 2) / f; /* round(2^30 / j!) */
	}
	LN2_Q16 = llround(log(2.0) * 65536.0);
	PI_Q16 = llround(M_PI * 65536.0);
	TWO_PI_Q16 = llround(2.0 * M_PI * 65536.0);
	HALF_PI_Q16 = llround(M_PI / 2.0 * 65536.0);
	GELU_A = llround(0.044715 * 65536.0);
	GELU_B = llround(0.7978845608 * 65536.0);
	EPS_Q32 = llround(1e-6 * 4294967296.0);
	EXP_HI = llround(log(32768.0) * 65536.0); /* exp(x) >= 32768 beyond this */
}

static int32_t expq(int32_t x)
{
	if (x > EXP_HI) return MAXV;
	if (x < -12 * 65536) return 0; /* exp(-12) < 2^-16 */
	const int64_t ln2 = LN2_Q16;
	int64_t k = x >= 0 ? x / ln2 : -((-(int64_t)x + ln2 - 1) / ln2);
	int64_t r = ((int64_t)x - k * ln2) * 16384; /* Q30 in [0, ln 2) */
	int64_t p = EXPC[8];
	for (int i = 7; i >= 0; i--) p = EXPC[i] + asr(p * r, 30);
	int sh = (int)k - 14;
	int64_t v = sh >= 0 ? p * ((int64_t)1 << sh) : asr(p + ((int64_t)1 << (-sh - 1)), -sh);
	return sat(v);
}

static int32_t logq(int32_t x)
{
	if (x <= 0) return MINV;
	int e = 0;
	uint32_t m = (uint32_t)x;
	while (m >= 131072u) {
		m >>= 1;
		e++;
	}
	while (m < 65536u) {
		m <<= 1;
		e--;
	}
	int64_t s = ((int64_t)(m - 65536) << 30) / (m + 65536), s2 = asr(s * s, 30), t = s, acc = 0;
	for (int k = 1; k <= 13; k += 2) {
		acc += t / k;
		t = asr(t * s2, 30);
	}
	return sat(asr(2 * acc, 14) + (int64_t)e * LN2_Q16);
}

static uint64_t isqrt64(uint64_t v)
{
	uint64_t r = 0, bit = (uint64_t)1 << 62;
	while (bit > v) bit >>= 2;
	while (bit) {
		if (v >= r + bit) {
			v -= r + bit;
			r = (r >> 1) + bit;
		} else {
			r >>= 1;
		}
		bit >>= 2;
	}
	return r;
}

static int32_t sinq(int32_t x)
{
	const int64_t pi = PI_Q16, two_pi = TWO_PI_Q16, half_pi = HALF_PI_Q16;
	int64_t r = (int64_t)x % two_pi;
	if (r > pi) r -= two_pi;
	if (r < -pi) r += two_pi;
	if (r > half_pi) r = pi - r;
	if (r < -half_pi) r = -pi - r;
	int64_t z = r * 16384, z2 = asr(z * z, 30), t = z, acc = 0;
	for (int k = 1; k <= 13; k += 2) {
		acc += t;
		t = -asr(t * z2, 30) / ((k + 1) * (k + 2));
	}
	return sat(asr(acc + 8192, 14));
}

static int32_t tanhq(int32_t x)
{
	int32_t t = absq(x);
	if (t > 9 * ONE) return x < 0 ? -ONE : ONE;
	int32_t e = expq(-2 * t);
	int32_t y = fdiv(ONE - e, ONE + e);
	return x < 0 ? -y : y;
}

static int32_t sigmoidq(int32_t x)
{
	int32_t e = expq(-absq(x));
	return x >= 0 ? fdiv(ONE, ONE + e) : fdiv(e, ONE + e);
}

int32_t tgo_to_fixed(double v, int frac)
{
	double s = v * (double)(1LL << frac);
	if (s >= 2147483647.0) return MAXV;
	if (s <= -2147483648.0) return MINV;
	return (int32_t)llround(s);
}

void tgo_to_fixed_rows(const float *in, int32_t *out, long n)
{
	for (long i = 0; i < n; i++) out[i] = tgo_to_fixed((double)in[i], 16);
}

/* 6-decimal text of a Q16.16 value (tg_rtq.h:403-418 restated). */
const char *tgo_fx_format(int32_t v, char *buf)
{
	int64_t x = v, neg = x < 0;
	if (neg) x = -x;
	int64_t ip = x >> 16, fr = ((x & 0xffff) * 1000000 + 32768) >> 16;
	if (fr >= 1000000) {
		ip++;
		fr -= 1000000;
	}
	char t[24];
	int n = 0;
	for (int i = 0; i < 6; i++) {
		t[n++] = (char)('0' + fr % 10);
		fr /= 10;
	}
	t[n++] = '.';
	do {
		t[n++] = (char)('0' + ip % 10);
		ip /= 10;
	} while (ip);
	if (neg) t[n++] = '-';
	int k = 0;
	while (n) buf[k++] = t[--n];
	buf[k] = 0;
	return buf;
}

int tgo_prepare_fixed(tgo_module *m)
{
	init_consts();
	if (m->fixed_ready) return 0;
	for (int v = 0; v < m->nval; v++) {
		tgo_value *x = &m->val[v];
		if (x->kind != TGO_PARAM && x->kind != TGO_STATE) continue;
		x->fx = malloc((size_t)x->n * sizeof *x->fx);
		if (!x->fx) return -1;
		for (long i = 0; i < x->n; i++) x->fx[i] = tgo_to_fixed((double)x->data[i], 16);
		if (x->qbits) {
			int nch = x->sh.dim[x->qaxis];
			x->fqs = malloc((size_t)nch * sizeof *x->fqs);
			if (!x->fqs) return -1;
			for (int i = 0; i < nch; i++) x->fqs[i] = tgo_to_fixed((double)x->qs[i], 24);
		}
	}
	m->fixed_ready = 1;
	return 0;
}

typedef struct {
	const tgo_module *m;
	int32_t *arena;
	const int32_t *in;
	int *steps;
} VM;

static int32_t *ptr(VM *vm, int v)
{
	const tgo_value *x = &vm->m->val[v];
	if (x->kind == TGO_PARAM || x->kind == TGO_STATE) return x->fx;
	if (x->kind == TGO_INPUT) {
		long off = 0;
		for (int i = 0; i < x->index; i++) off += vm->m->val[vm->m->inputs[i]].n;
		return (int32_t *)vm->in + off;
	}
	return vm->arena + x->off;
}

static int32_t bop(int op, int32_t x, int32_t y)
{
	switch (op) {
	case O_ADD: return sat((int64_t)x + y);
	case O_SUB: return sat((int64_t)x - y);
	case O_MUL: return fmul(x, y);
	case O_DIV: return fdiv(x, y);
	case O_MAX: return x > y ? x : y;
	default: return x < y ? x : y;
	}
}

static void kbin(int op, int32_t *o, const int32_t *a, int sa, const int32_t *b, int sb, int n)
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

static void bin(VM *vm, const tgo_ins *in, int32_t *o, const int32_t *a, const int32_t *b)
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

static int32_t un(int op, int32_t x)
{
	switch (op) {
	case O_NEG: return sat(-(int64_t)x);
	case O_TANH: return tanhq(x);
	case O_RELU: return x > 0 ? x : 0;
	case O_SIGMOID: return sigmoidq(x);
	case O_EXP: return expq(x);
	case O_SQRT: return x > 0 ? (int32_t)isqrt64((uint64_t)x << 16) : 0;
	case O_GELU: {
		int64_t v = x, x3 = asr(asr(v * v, 16) * v, 16);
		int64_t u = asr((v + asr(x3 * GELU_A, 16)) * GELU_B, 16);
		int32_t t = tanhq(sat(u));
		return sat(asr(v * ((int64_t)ONE + t), 17));
	}
	case O_SILU: return fmul(x, sigmoidq(x));
	case O_SOFTPLUS: return sat((int64_t)(x > 0 ? x : 0) + logq(ONE + expq(-absq(x))));
	case O_LOG: return logq(x);
	case O_SIN: return sinq(x);
	case O_COS: return sinq(sat((int64_t)x + HALF_PI_Q16));
	case O_FLOOR: return (int32_t)((uint32_t)x & 0xffff0000u);
	default: return x > 0 ? ONE : 0; /* step */
	}
}

static int32_t qscale(int64_t acc, int32_t s24)
{
	int64_t p = (int64_t)((uint64_t)acc * (uint64_t)(int64_t)s24); /* wraps like the reference's int64 product */
	return sat(asr(p + ((int64_t)1 << 23), 24));
}

static int32_t delta(const int32_t *a, const int32_t *b, int n)
{
	int32_t d = 0;
	for (int i = 0; i < n; i++) {
		int32_t e = absq(sat((int64_t)a[i] - b[i]));
		if (e > d) d = e;
	}
	return d;
}

static void copy(int32_t *o, const int32_t *a, long n)
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
	int32_t *o = ptr(vm, in->out);
	int n = m->val[in->out].n;
	const int32_t *a = in->na > 0 ? ptr(vm, in->a[0]) : NULL;
	const int32_t *c = in->na > 1 ? ptr(vm, in->a[1]) : NULL;
	switch (in->op) {
	case O_CONST: o[0] = tgo_to_fixed((double)in->k, 16); break;
	case O_ADD: case O_SUB: case O_MUL: case O_DIV: case O_MAX: case O_MIN: bin(vm, in, o, a, c); break;
	case O_NEG: case O_TANH: case O_RELU: case O_SIGMOID: case O_EXP: case O_SQRT: case O_GELU: case O_SILU:
	case O_SOFTPLUS: case O_LOG: case O_SIN: case O_COS: case O_FLOOR: case O_STEP:
		for (int i = 0; i < n; i++) o[i] = un(in->op, a[i]);
		break;
	case O_MATMUL: {
		int mm, kk, nn, gg;
		const tgo_value *qa = &m->val[in->a[0]], *qb = &m->val[in->a[1]];
		tgo_matmul_dims(&qa->sh, &qb->sh, &mm, &kk, &nn, &gg);
		int mode = 0; /* 0 plain, 1 quantized left (axis 0), 2 quantized right (axis 1) */
		if (gg == 1 && qa->qbits && tgo_q_axis_for(m, in->a[0], in) == qa->qaxis) mode = 1;
		else if (gg == 1 && qb->qbits && tgo_q_axis_for(m, in->a[1], in) == qb->qaxis) mode = 2;
		for (int g = 0; g < gg; g++) {
			const int32_t *ag = a + (long)g * mm * kk, *bg = c + (long)g * kk * nn;
			int32_t *og = o + (long)g * mm * nn;
			for (int i = 0; i < mm; i++)
				for (int j = 0; j < nn; j++) {
					int64_t s = 0;
					if (mode == 1) {
						for (int p = 0; p < kk; p++) s += (int64_t)tgo_qget(qa->q, qa->qbits, (long)i * kk + p) * bg[(long)p * nn + j];
						og[(long)i * nn + j] = qscale(s, qa->fqs[i]);
					} else if (mode == 2) {
						for (int p = 0; p < kk; p++) s += (int64_t)ag[(long)i * kk + p] * tgo_qget(qb->q, qb->qbits, (long)p * nn + j);
						og[(long)i * nn + j] = qscale(s, qb->fqs[j]);
					} else {
						for (int p = 0; p < kk; p++) s += (int64_t)ag[(long)i * kk + p] * bg[(long)p * nn + j];
						og[(long)i * nn + j] = sat(asr(s + 32768, 16));
					}
				}
		}
		break;
	}
	case O_SOFTMAX:
	case O_RMSNORM: {
		const tgo_shape *s = &m->val[in->a[0]].sh;
		int cols = s->rank ? s->dim[s->rank - 1] : 1, rows = tgo_numel(s) / cols;
		for (int r = 0; r < rows; r++) {
			const int32_t *x = a + (long)r * cols;
			int32_t *y = o + (long)r * cols;
			if (in->op == O_SOFTMAX) {
				int32_t mx = x[0];
				int64_t sum = 0;
				for (int i = 1; i < cols; i++)
					if (x[i] > mx) mx = x[i];
				for (int i = 0; i < cols; i++) {
					y[i] = expq(sat((int64_t)x[i] - mx));
					sum += y[i];
				}
				for (int i = 0; i < cols; i++) y[i] = (int32_t)(((int64_t)y[i] * 65536 + sum / 2) / sum);
			} else {
				uint64_t ss = 0;
				for (int i = 0; i < cols; i++) ss += (uint64_t)((int64_t)x[i] * x[i]);
				uint64_t ms = ss / (uint64_t)cols + (uint64_t)EPS_Q32;
				int32_t rms = (int32_t)isqrt64(ms);
				for (int i = 0; i < cols; i++) y[i] = fdiv(x[i], rms > 0 ? rms : 1);
			}
		}
		break;
	}
	case O_SUM:
	case O_MEAN: {
		int k = m->val[in->a[0]].n;
		int64_t s = 0;
		for (int i = 0; i < k; i++) s += a[i];
		o[0] = in->op == O_SUM ? sat(s) : sat(s / k);
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
			for (int j = 0; j < nn; j++) o[(long)i * nn + j] = fmul(a[i], c[j]);
		break;
	}
	case O_RESHAPE: copy(o, a, n); break;
	case O_TAKE: {
		const tgo_shape *s0 = &m->val[in->a[0]].sh;
		int cnt = m->val[in->a[1]].sh.dim[0], d = s0->dim[0], h = tgo_numel(s0) / s0->dim[0];
		for (int i = 0; i < cnt; i++) {
			int64_t rr = asr((int64_t)c[i] + 32768, 16);
			int t = rr >= 0 && rr < d ? (int)rr : -1;
			for (int j = 0; j < h; j++) o[(long)i * h + j] = t >= 0 ? a[(long)t * h + j] : 0;
		}
		break;
	}
	case O_THINK: {
		copy(o, ptr(vm, in->init), n);
		int32_t thr = 0;
		if (in->eps >= 0) {
			thr = tgo_to_fixed((double)in->eps, 16);
			if (!(thr > 0 || in->eps == 0)) thr = 1; /* a positive threshold stays positive */
		}
		int32_t sv = ONE, hthr = tgo_to_fixed((double)in->hthr, 16);
		int it = 0;
		while (it < in->maxit) {
			exec(vm, in->body);
			it++;
			const int32_t *y = ptr(vm, in->yield);
			int32_t d = delta(y, o, n);
			copy(o, y, n);
			if (in->eps >= 0 && (tgo_plant == 1 ? d < thr : tgo_plant == 2 ? d <= thr - 1 : d <= thr)) break;
			if (in->halt >= 0) {
				int32_t h = *ptr(vm, in->halt), p = h < 0 ? 0 : h > ONE ? ONE : h;
				sv = fmul(sv, ONE - p);
				if (ONE - sv > hthr) break;
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

void tgo_run_row_fixed(const tgo_module *m, const int32_t *in, int32_t *out, int *steps, int32_t *arena)
{
	VM vm = { m, arena, in, steps };
	exec(&vm, &m->top);
	copy(out, ptr(&vm, m->output), m->nout);
}

/* Test access to the scalar primitives (op: 0 fmul, 1 fdiv, 2 expq, 3 logq,
 * 4 isqrt64, 5 sinq, 6 tanhq, 7 sigmoidq, 8 exp polynomial coefficient a). */
int64_t tgo_fx_prim(int op, int64_t a, int64_t b)
{
	init_consts();
	switch (op) {
	case 0: return fmul((int32_t)a, (int32_t)b);
	case 1: return fdiv((int32_t)a, (int32_t)b);
	case 2: return expq((int32_t)a);
	case 3: return logq((int32_t)a);
	case 4: return (int64_t)isqrt64((uint64_t)a);
	case 5: return sinq((int32_t)a);
	case 6: return tanhq((int32_t)a);
	case 7: return sigmoidq((int32_t)a);
	case 8: return a >= 0 && a <= 8 ? EXPC[a] : 0;
	}
	return 0;
}
