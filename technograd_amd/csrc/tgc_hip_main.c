/* tgc-hip: `tgc batch` on the MI355X backend.
 *
 *   tgc-hip batch MODEL DATA [-o OUT] [--fixed] [--exact] [--rows N] [-v] [--log FILE]
 *
 * Same input/output contract as the reference's batch command
 * (src/main.c:400-444, src/io.c): DATA is raw little-endian f32 when it ends in
 * .bin or .f32, otherwise text rows of numbers separated by commas or blanks
 * with `#` comments (src/io.c:23-41); every row is validated before anything
 * is computed or the output file is created; rows run in blocks (device
 * passes of up to --rows rows) and each block is written, in input order, as
 * soon as it is done: text as %.9g with the steps of every think loop
 * appended (src/io.c:79-93), binary as raw f32 without steps. SIGINT or
 * SIGTERM stops the batch after the current block and the exit status is
 * 128 + the signal number (src/main.c:418, :431, :444; src/serve.c:49-69).
 * Stateful models and models outside the backend are refused with a message
 * (the reference CLI runs those).
 *
 * --fixed runs the model in Q16.16 (the number system of `tgc c --fixed`
 * units): text inputs are read with the exact decimal rule of tg_fx_parse
 * (runtime/tg_rtq.h:375-401: integer digits kept up to the first value of at
 * least 100000, at most 12 fraction digits, an optional exponent, the
 * rational value rounded half away from zero to 1/65536 and saturated),
 * binary inputs by rounding x * 2^16 half away from zero; text outputs are
 * printed with 6 decimals (tg_fx_format, :403-418) and binary outputs are
 * the exact f32 values q / 65536.
 *
 * The environment variable TGC_HIP_TEST_SIGTERM_AFTER_BLOCKS=N makes the
 * program send itself SIGTERM after N blocks (tests of the stop path).
 *
 * -v prints the batch summary of src/main.c:155-173 on stderr; --log FILE
 * appends it as JSON Lines events (`batch`, then `think` per loop), the
 * reference's trace format (src/trace.c: t, level, stage, msg, fields).
 *
 *   tgc-hip fxparse TOKEN...   prints each token's Q16.16 value (no device)
 *   tgc-hip stream MODEL [SRC] [-o DST] [--fixed] [--exact] [--rows N]
 *   tgc-hip serve MODEL --listen [HOST:]PORT [--fixed] [--exact] [--rows N] [--window-us U]
 *       the reference's connections (src/serve.c) on the device batch: see tgc_hip_serve.c
 *   tgc-hip ir MODEL.tg
 *       prints the canonical TGIR of a surface model (no device)
 *   tgc-hip quantize MODEL [-o OUT.tgir] [--bits 8|4] [--method rtn|gptq] [--calib DATA] [--min-size N] [--max-k K]
 *       `tgc quantize` with the calibration run and Hessians on the device;
 *       --max-k (default 2048, the reference's limit) bounds the layer width
 *       given a Hessian, 0 gives every layer one
 *   tgc-hip c MODEL [--fixed] [-o UNIT.hip] [--kernel NAME]
 *       writes the model's row program as a freestanding HIP unit (the
 *       device counterpart of `tgc c`, src/main.c:343-360; no device)
 */
#include "tg_hip.h"
#include "tgc_hip_cli.h"

#include <math.h>
#include <pthread.h>
#include <signal.h>
#include <stdatomic.h>
#include <stdint.h>
#include <ctype.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* the signal that asked the batch to stop (0: none) */
static atomic_int stop_sig;
static void on_signal(int sig) { atomic_store(&stop_sig, sig); }
int stop_signal(void) { return atomic_load(&stop_sig); }

void install_signals(void)
{
	struct sigaction sa;
	memset(&sa, 0, sizeof sa);
	sa.sa_handler = on_signal;
	sigemptyset(&sa.sa_mask);
	sigaction(SIGINT, &sa, NULL);
	sigaction(SIGTERM, &sa, NULL);
	signal(SIGPIPE, SIG_IGN);
}

/* Decimal text to Q16.16 (the reference's tg_fx_parse, runtime/tg_rtq.h:375-401),
 * in two stages: fx_lex reads the token's parts, fx_value turns them into the
 * Q16.16 word. The observable rule: an optional sign; integer digits, of
 * which only those read while the integer part is below 100000 count;
 * fraction digits, of which only the first twelve count; an optional
 * exponent; the value num / den with num = int * 10^f + frac and den = 10^f,
 * num scaled by 10 per positive exponent step until it passes 2^47 (later
 * steps are dropped), den by 10 per negative step; q = (num * 65536 + den /
 * 2) / den. The products are 64-bit and wrap. The reference's build assumes
 * they cannot, and so keeps one saturation bound per sign: a positive token's
 * q is clamped above and otherwise truncated to 32 bits, a negative token's
 * -q clamped below and otherwise truncated (tests/golden/fx_parse.json holds
 * tokens whose products wrap). The exponent's digits accumulate in 32 bits
 * with wrap-around, and the same assumption (that they cannot wrap) decides
 * what a wrapped exponent does there: without a '-' it scales only when its
 * signed 32-bit value is positive; with a '-' den is scaled as many times as
 * its unsigned value says (den wraps to 0 within 64 steps, where the
 * reference's division traps and this parser gives 0). */
typedef struct {
	int neg, digits, eneg;
	uint32_t ex; /* the exponent's digits, accumulated modulo 2^32 */
	int64_t ip, fn, fd;
} FxParts;

static const char *fx_lex(const char *s, FxParts *t)
{
	memset(t, 0, sizeof *t);
	t->fd = 1;
	if (*s == '-' || *s == '+') t->neg = *s++ == '-';
	for (; isdigit((unsigned char)*s); s++, t->digits++)
		if (t->ip < 100000) t->ip = t->ip * 10 + (*s - '0');
	if (*s == '.')
		for (s++; isdigit((unsigned char)*s); s++, t->digits++)
			if (t->fd < 1000000000000LL) t->fn = t->fn * 10 + (*s - '0'), t->fd *= 10;
	if (*s == 'e' || *s == 'E') {
		s++;
		t->eneg = *s == '-';
		if (*s == '-' || *s == '+') s++;
		for (; isdigit((unsigned char)*s); s++) t->ex = t->ex * 10u + (uint32_t)(*s - '0');
	}
	return s;
}

static int32_t low32(int64_t x) { return (int32_t)(uint32_t)(uint64_t)x; }

static int32_t fx_value(const FxParts *t)
{
	int64_t num = t->ip * t->fd + t->fn; /* below 10^18 */
	uint64_t den = (uint64_t)t->fd;
	if (!t->eneg && t->ex <= (uint32_t)INT32_MAX) /* (zero stays zero) */
		for (uint32_t k = t->ex; k && num && num <= ((int64_t)1 << 47); k--) num *= 10;
	if (t->eneg)
		for (uint32_t k = t->ex; k && den; k--) den *= 10u; /* wraps modulo 2^64, to 0 within 64 steps */
	const int64_t d = (int64_t)den;
	if (d == 0 || d == -1) return 0; /* a divisor the reference's division would trap on */
	const int64_t q = (int64_t)((uint64_t)num * 65536u + (uint64_t)(d / 2)) / d;
	if (!t->neg) return q > INT32_MAX ? INT32_MAX : low32(q);
	const int64_t v = (int64_t)(0u - (uint64_t)q);
	return v < INT32_MIN ? INT32_MIN : low32(v);
}

/* the token at s as Q16.16 into *v; its end, or NULL when it has no digits */
static const char *fx_parse(const char *s, int32_t *v)
{
	FxParts t;
	const char *e = fx_lex(s, &t);
	if (!t.digits) return NULL;
	*v = fx_value(&t);
	return e;
}

int die(const char *fmt, const char *a)
{
	fprintf(stderr, "tgc-hip: error: ");
	fprintf(stderr, fmt, a);
	fputc('\n', stderr);
	return 1;
}

static int is_binary(const char *path)
{
	const char *dot = strrchr(path, '.');
	return dot && (!strcmp(dot, ".bin") || !strcmp(dot, ".f32"));
}

static char *slurp(const char *path, size_t *len)
{
	FILE *f = strcmp(path, "-") ? fopen(path, "rb") : stdin;
	if (!f) return NULL;
	size_t cap = 1 << 16, n = 0;
	char *b = malloc(cap + 1);
	for (;;) {
		if (n == cap) b = realloc(b, (cap *= 2) + 1);
		size_t k = fread(b + n, 1, cap - n, f);
		if (!k) break;
		n += k;
	}
	if (f != stdin) fclose(f);
	b[n] = 0;
	*len = n;
	return b;
}

/* The text row format (src/io.c:25-41): numbers separated by blanks or
 * commas, the rest of the line after '#' a comment. A token must end at a
 * separator, a comment or the line's end. */
static int row_sep(char c) { return c == ' ' || c == '\t' || c == ',' || c == '\r' || c == '\n'; }

/* one number at s into *x (f32, or a Q16.16 word's bits); its end (s itself if none) */
static const char *row_token(const char *s, float *x, int fixed)
{
	if (!fixed) {
		char *e;
		*x = strtof(s, &e);
		return e;
	}
	int32_t q = 0;
	const char *e = fx_parse(s, &q);
	memcpy(x, &q, 4);
	return e ? e : s;
}

/* the numbers of one text line, up to max kept in v; their count, or -1
 * with *bad at the first token that is not a number */
int parse_row(const char *s, float *v, int max, const char **bad, int fixed)
{
	int n = 0;
	for (;;) {
		while (row_sep(*s)) s++;
		if (!*s || *s == '#') return n;
		float x;
		const char *e = row_token(s, &x, fixed);
		if (e == s || !(*e == 0 || *e == '#' || row_sep(*e))) {
			*bad = s;
			return -1;
		}
		if (n < max) v[n] = x;
		n++;
		s = e;
	}
}

static int host_is_le(void)
{
	const uint32_t one = 1;
	unsigned char b;
	memcpy(&b, &one, 1);
	return b == 1;
}

/* Row, output and step buffers: pinned host memory where the library can give
 * it (tg_hip_batch then moves them over PCIe without a staging copy), else
 * ordinary memory; *pinned says which, for host_buf_free. */
static void *host_buf(size_t bytes, int *pinned)
{
	void *p = tg_hip_host_alloc(bytes ? bytes : 4);
	*pinned = p != NULL;
	return p ? p : malloc(bytes ? bytes : 4);
}

static void host_buf_free(void *p, int pinned)
{
	if (pinned) tg_hip_host_free(p);
	else free(p);
}

/* a binary row file (raw little-endian f32) read straight into a row buffer */
static float *load_binary_rows(const char *path, int per, long *rows, char *err, size_t errn, int *pinned)
{
	FILE *f = fopen(path, "rb");
	long len = -1;
	if (f && !fseek(f, 0, SEEK_END)) len = ftell(f);
	if (len < 0 || fseek(f, 0, SEEK_SET)) {
		snprintf(err, errn, "cannot read '%s'", path);
		if (f) fclose(f);
		return NULL;
	}
	if (len % 4 || (len / 4) % per) {
		snprintf(err, errn, "'%s': %ld bytes is not a whole number of %d-float rows", path, len, per);
		fclose(f);
		return NULL;
	}
	float *all = host_buf((size_t)len, pinned);
	const size_t got = all ? fread(all, 1, (size_t)len, f) : 0;
	fclose(f);
	if (!all || got != (size_t)len) {
		snprintf(err, errn, "cannot read '%s'", path);
		if (all) host_buf_free(all, *pinned);
		return NULL;
	}
	if (!host_is_le()) /* the file is little-endian */
		for (long i = 0; i < len / 4; i++) {
			const unsigned char *b = (const unsigned char *)&all[i];
			const uint32_t w = (uint32_t)b[0] | (uint32_t)b[1] << 8 | (uint32_t)b[2] << 16 | (uint32_t)b[3] << 24;
			memcpy(&all[i], &w, 4);
		}
	*rows = len / 4 / per;
	return all;
}

/* every row of DATA: f32 values, or with `fixed` Q16.16 words (binary inputs
 * are f32 either way; the caller converts them), in a row buffer (host_buf) */
static float *load_rows(const char *path, int per, long *rows, char *err, size_t errn, int fixed, int *pinned)
{
	if (is_binary(path)) return load_binary_rows(path, per, rows, err, errn, pinned);
	size_t len;
	char *raw = slurp(path, &len);
	if (!raw) {
		snprintf(err, errn, "cannot read '%s'", path);
		return NULL;
	}
	float *all = NULL;
	*pinned = 0;
	long n = 0;
	for (int pass = 0; pass < 2; pass++) { /* pass 0 validates and counts, pass 1 parses */
		if (pass) all = host_buf((size_t)(n ? n : 1) * per * sizeof *all, pinned);
		long r = 0;
		int line = 1;
		for (char *s = raw; *s; line++) {
			char *nl = strchr(s, '\n');
			if (nl) *nl = 0;
			const char *bad;
			int k = parse_row(s, NULL, 0, &bad, fixed);
			if (k < 0) {
				snprintf(err, errn, "%s:%d: bad number near '%.20s'", path, line, bad);
				free(raw);
				if (all) host_buf_free(all, *pinned);
				return NULL;
			}
			if (k > 0 && k != per) {
				snprintf(err, errn, "%s:%d: row has %d values, the model needs %d", path, line, k, per);
				free(raw);
				if (all) host_buf_free(all, *pinned);
				return NULL;
			}
			if (k > 0) {
				if (pass) parse_row(s, all + (size_t)r * per, per, &bad, fixed);
				r++;
			}
			if (nl) *nl = '\n';
			if (!nl) break;
			s = nl + 1;
		}
		n = r;
	}
	free(raw);
	*rows = n;
	return all;
}

void fx_format(int32_t v, char *buf) /* 6 decimals, integer arithmetic */
{
	int64_t x = v, neg = x < 0;
	if (neg) x = -x;
	int64_t ip = x >> 16, fr = ((x & 0xffff) * 1000000 + 32768) >> 16;
	if (fr >= 1000000) {
		ip++;
		fr -= 1000000;
	}
	sprintf(buf, "%s%lld.%06lld", neg ? "-" : "", (long long)ip, (long long)fr);
}

static double now_ms(void)
{
	struct timespec t;
	clock_gettime(CLOCK_MONOTONIC, &t);
	return t.tv_sec * 1e3 + t.tv_nsec / 1e6;
}

/* one JSON Lines event in the reference's trace format: t, level, stage, msg,
 * then `fields` (already JSON text, starting with a comma) */
static void log_event(FILE *lf, const char *stage, const char *msg, const char *fields)
{
	if (!lf) return;
	struct timespec ts;
	timespec_get(&ts, TIME_UTC);
	fprintf(lf, "{\"t\":%.3f,\"level\":\"info\",\"stage\":\"%s\",\"msg\":\"%s\"%s}\n", (double)ts.tv_sec + ts.tv_nsec / 1e9, stage,
		msg, fields);
	fflush(lf);
}

static void write_block(FILE *f, int obin, int fixed, const float *out, const int *steps, long n, int nout, int nthink, int nt)
{
	char buf[32];
	if (obin && !fixed && host_is_le()) { /* raw f32, the memory's own bytes */
		fwrite(out, 4, (size_t)n * nout, f);
		return;
	}
	for (long r = 0; r < n; r++) {
		const float *y = out + (size_t)r * nout;
		if (obin) {
			for (int i = 0; i < nout; i++) {
				float v = y[i];
				if (fixed) {
					int32_t q;
					memcpy(&q, &y[i], 4);
					v = (float)((double)q / 65536.0);
				}
				uint32_t w;
				memcpy(&w, &v, 4);
				unsigned char b[4] = { (unsigned char)w, (unsigned char)(w >> 8), (unsigned char)(w >> 16), (unsigned char)(w >> 24) };
				fwrite(b, 1, 4, f);
			}
			continue;
		}
		for (int i = 0; i < nout; i++) {
			if (fixed) {
				int32_t q;
				memcpy(&q, &y[i], 4);
				fx_format(q, buf);
				fprintf(f, "%s%s", i ? "," : "", buf);
			} else {
				fprintf(f, "%s%.9g", i ? "," : "", (double)y[i]);
			}
		}
		for (int t = 0; t < nthink; t++) fprintf(f, ",%d", steps[(size_t)r * nt + t]);
		fputc('\n', f);
	}
}

/* a model file's TGIR: the file itself, or a surface (.tg) model lowered
 * (the reference's load_module rule, src/util.c:335-369: TGIR starts with
 * '(' or ';' after blanks); NULL with the reason in err */
char *load_model(const char *path, size_t *len, char *err, size_t errn)
{
	char *text = slurp(path, len);
	if (!text) {
		snprintf(err, errn, "cannot read '%s'", path);
		return NULL;
	}
	const char *c = text;
	while (*c == ' ' || *c == '\t' || *c == '\n' || *c == '\r') c++;
	if (*c == '(' || *c == ';') return text;
	free(text);
	char *t = tg_hip_surface_to_tgir(path);
	if (!t) {
		snprintf(err, errn, "%s", tg_hip_error());
		return NULL;
	}
	*len = strlen(t);
	char *r = malloc(*len + 1);
	if (r) memcpy(r, t, *len + 1);
	else snprintf(err, errn, "out of memory");
	tg_hip_str_free(t);
	return r;
}

/* tgc-hip ir MODEL.tg: the canonical TGIR of a surface model (src/main.c:373-375) */
static int print_ir(int argc, char **argv)
{
	if (argc != 3) return die("usage: tgc-hip ir MODEL.tg%s", "");
	char *t = tg_hip_surface_to_tgir(argv[2]);
	if (!t) return die("%s", tg_hip_error());
	fputs(t, stdout);
	tg_hip_str_free(t);
	return fflush(stdout) ? die("cannot write the TGIR%s", "") : 0;
}

/* tgc-hip c: the row program as a HIP unit (tg_hip_emit_unit) */
static int emit_unit(int argc, char **argv)
{
	const char *model = NULL, *opath = NULL, *kernel = NULL;
	int flags = 0;
	for (int i = 2; i < argc; i++) {
		if (!strcmp(argv[i], "-o") && i + 1 < argc) opath = argv[++i];
		else if (!strcmp(argv[i], "--kernel") && i + 1 < argc) kernel = argv[++i];
		else if (!strcmp(argv[i], "--fixed")) flags |= TG_HIP_FIXED;
		else if (!model) model = argv[i];
		else return die("unexpected argument '%s'", argv[i]);
	}
	if (!model) return die("usage: tgc-hip c MODEL.tgir [--fixed] [-o UNIT.hip] [--kernel NAME]%s", "");
	size_t mlen;
	char lerr[1024];
	char *text = load_model(model, &mlen, lerr, sizeof lerr);
	if (!text) return die("%s", lerr);
	char *src = tg_hip_emit_unit(text, mlen, flags, kernel);
	free(text);
	if (!src) return die("%s", tg_hip_error());
	FILE *f = opath ? fopen(opath, "w") : stdout;
	if (!f) {
		tg_hip_str_free(src);
		return die("cannot open '%s'", opath);
	}
	const size_t n = strlen(src);
	const int ok = fwrite(src, 1, n, f) == n;
	tg_hip_str_free(src);
	if (opath && fclose(f)) return die("cannot write '%s'", opath);
	return ok ? 0 : die("cannot write the unit%s", "");
}

/* tgc-hip quantize: `tgc quantize` (src/quant.c:318-384) with the calibration
 * run and the Hessians on the device (tg_hip_quantize_model) */
#define QUSAGE "usage: tgc-hip quantize MODEL [-o OUT.tgir] [--bits 8|4] [--method rtn|gptq] [--calib DATA] [--min-size N] [--max-k K]%s"
static int quantize(int argc, char **argv)
{
	const char *src = NULL, *opath = NULL, *calib = NULL, *method = "rtn";
	int bits = 8, min_size = 256, max_k = 2048;
	for (int i = 2; i < argc; i++) {
		const char *a = argv[i];
		const int v = i + 1 < argc;
		if (!strcmp(a, "-o") && v) opath = argv[++i];
		else if (!strcmp(a, "--bits") && v) bits = atoi(argv[++i]);
		else if (!strcmp(a, "--method") && v) method = argv[++i];
		else if (!strcmp(a, "--calib") && v) calib = argv[++i];
		else if (!strcmp(a, "--min-size") && v) min_size = atoi(argv[++i]);
		else if (!strcmp(a, "--max-k") && v) max_k = atoi(argv[++i]);
		else if (!src && a[0] != '-') src = a;
		else return die(QUSAGE, "");
	}
	if (!src) return die(QUSAGE, "");
	if (bits != 8 && bits != 4) return die("--bits is 8 or 4%s", "");
	const int gptq = !strcmp(method, "gptq");
	if (!gptq && strcmp(method, "rtn")) return die("--method is rtn or gptq%s", "");
	if (gptq && !calib) return die("--method gptq needs --calib DATA (input rows in the tgc batch format)%s", "");
	size_t mlen;
	char lerr[1024];
	char *text = load_model(src, &mlen, lerr, sizeof lerr);
	if (!text) return die("%s", lerr);
	float *rows = NULL;
	long nrows = 0;
	int rows_pinned = 0;
	if (calib) { /* the rows' width comes from the model on the device */
		if (tg_hip_init(0)) return die("%s", tg_hip_error());
		tg_hip_prog *p = tg_hip_load(text, mlen, 0, 1);
		if (!p) return die("%s", tg_hip_error());
		int per, nout, nthink;
		tg_hip_info(p, &per, &nout, &nthink);
		tg_hip_free(p);
		rows = load_rows(calib, per, &nrows, lerr, sizeof lerr, 0, &rows_pinned);
		if (!rows) return die("%s", lerr);
		if (!nrows) return die("%s: no calibration rows", calib);
	}
	static char log[1 << 16];
	long bytes[2];
	char *out = tg_hip_quantize_model(text, mlen, bits, gptq, rows, nrows, min_size, max_k, bytes, log, sizeof log);
	free(text);
	if (rows) host_buf_free(rows, rows_pinned);
	fputs(log, stderr);
	if (!out) return die("%s", tg_hip_error());
	char dflt[1024];
	if (!opath) {
		const char *dot = strrchr(src, '.');
		snprintf(dflt, sizeof dflt, "%.*s.q%d.tgir", (int)(dot ? dot - src : (long)strlen(src)), src, bits);
		opath = dflt;
	}
	FILE *f = fopen(opath, "w");
	if (!f) {
		tg_hip_str_free(out);
		return die("cannot write '%s'", opath);
	}
	const size_t n = strlen(out);
	const int ok = fwrite(out, 1, n, f) == n;
	tg_hip_str_free(out);
	if (fclose(f) || !ok) return die("write failed '%s'", opath);
	fprintf(stderr, "quantize: params %ld -> %ld bytes (%.1fx smaller); wrote %s\n", bytes[0], bytes[1],
		bytes[1] ? (double)bytes[0] / bytes[1] : 0.0, opath);
	return 0;
}

#define USAGE "usage: tgc-hip batch MODEL DATA [-o OUT] [--fixed] [--exact] [--rows N] [-v] [--log FILE]%s"

/* A batch in progress: the program, the output, and the summary of -v / --log. */
typedef struct {
	tg_hip_prog *p;
	int per, nout, nthink, nt, fixed, obin;
	FILE *f;
	long done, raise_after;
	long *ssum;
	int *smin, *smax;
	double dev_ms;
	char err[256];
} Run;

/* one device pass over n rows (f32, or Q16.16 words with `fixed`) and its think steps into the summary */
static int run_block(Run *r, const float *in, long n, float *out, int *steps)
{
	const int rc = r->fixed ? tg_hip_batch_fixed(r->p, (const int32_t *)in, n, (int32_t *)out, steps) : tg_hip_batch(r->p, in, n, out, steps);
	if (rc) return rc;
	tg_hip_stats_t st;
	tg_hip_stats(r->p, &st);
	r->dev_ms += st.batch_ms;
	for (int t = 0; t < r->nthink; t++)
		for (long i = 0; i < n; i++) {
			const int sv = steps[(size_t)i * r->nt + t];
			if (!r->done && !i) r->smin[t] = r->smax[t] = sv;
			r->ssum[t] += sv;
			r->smin[t] = sv < r->smin[t] ? sv : r->smin[t];
			r->smax[t] = sv > r->smax[t] ? sv : r->smax[t];
		}
	return 0;
}

/* n more rows written; at the end of a block, the test hook's stop request */
static void block_done(Run *r, long n, long block)
{
	r->done += n;
	if (r->raise_after > 0 && r->done % block == 0 && r->done / block == r->raise_after) raise(SIGTERM);
}

/* Raw f32 rows streamed from `in` through NSLOT pinned slots: a reader thread
 * fills a slot straight from the file (no staging copy), this thread runs the
 * slot's device pass, a writer thread writes its outputs, so the file's
 * reading and writing overlap the device. Chunks tile the blocks of `block`
 * rows, and a stop request ends the batch after the block it arrives in, as
 * the in-memory path does. Returns 0, or -1 with the reason in r->err (or
 * tg_hip_error()). */
enum { NSLOT = 3 };
typedef struct {
	Run *r;
	FILE *in;
	long rows, chunk, nch;
	float *in_b[NSLOT], *out_b[NSLOT];
	int *st_b[NSLOT];
	int pin[NSLOT][3];
	long n[NSLOT];
	int state[NSLOT]; /* 0 free, 1 rows read, 2 outputs computed */
	long last;        /* chunks the device has run: the reader and writer stop there */
	int quit;
	pthread_mutex_t mu;
	pthread_cond_t cv;
} Stream;

static void *stream_reader(void *arg)
{
	Stream *S = arg;
	const Run *r = S->r;
	for (long i = 0; i < S->nch; i++) {
		const int k = (int)(i % NSLOT);
		pthread_mutex_lock(&S->mu);
		while (S->state[k] != 0 && !S->quit) pthread_cond_wait(&S->cv, &S->mu);
		const int quit = S->quit;
		pthread_mutex_unlock(&S->mu);
		if (quit) break;
		const long n = S->rows - i * S->chunk < S->chunk ? S->rows - i * S->chunk : S->chunk;
		const size_t want = (size_t)n * r->per;
		const int ok = fread(S->in_b[k], 4, want, S->in) == want;
		if (ok && !host_is_le()) /* the file is little-endian */
			for (size_t j = 0; j < want; j++) {
				const unsigned char *b = (const unsigned char *)&S->in_b[k][j];
				const uint32_t w = (uint32_t)b[0] | (uint32_t)b[1] << 8 | (uint32_t)b[2] << 16 | (uint32_t)b[3] << 24;
				memcpy(&S->in_b[k][j], &w, 4);
			}
		if (ok && r->fixed) /* f32 rows: x * 2^16 rounded half away from zero, saturated */
			for (size_t j = 0; j < want; j++) {
				const double v = (double)S->in_b[k][j] * 65536.0;
				const int32_t q = v >= 2147483647.0 ? INT32_MAX : v <= -2147483648.0 ? INT32_MIN : (int32_t)llround(v);
				memcpy(&S->in_b[k][j], &q, 4);
			}
		pthread_mutex_lock(&S->mu);
		S->n[k] = ok ? n : -1;
		S->state[k] = 1;
		pthread_cond_broadcast(&S->cv);
		pthread_mutex_unlock(&S->mu);
		if (!ok) break;
	}
	return NULL;
}

static void *stream_writer(void *arg)
{
	Stream *S = arg;
	const Run *r = S->r;
	for (long i = 0;; i++) {
		const int k = (int)(i % NSLOT);
		pthread_mutex_lock(&S->mu);
		while (S->state[k] != 2 && !(S->quit && i >= S->last)) pthread_cond_wait(&S->cv, &S->mu);
		const int stop = S->state[k] != 2;
		pthread_mutex_unlock(&S->mu);
		if (stop) break;
		write_block(r->f, r->obin, r->fixed, S->out_b[k], S->st_b[k], S->n[k], r->nout, r->nthink, r->nt);
		pthread_mutex_lock(&S->mu);
		S->state[k] = 0;
		pthread_cond_broadcast(&S->cv);
		pthread_mutex_unlock(&S->mu);
	}
	return NULL;
}

static int stream_rows(Run *r, FILE *in, long rows, long block)
{
	Stream S;
	memset(&S, 0, sizeof S);
	S.r = r, S.in = in, S.rows = rows;
	const long target = (8l << 20) / (4l * (r->per > r->nout ? r->per : r->nout)); /* rows of about 8 MiB */
	const long per_block = (block + (target > 0 ? target : 1) - 1) / (target > 0 ? target : 1);
	S.chunk = (block + per_block - 1) / per_block; /* chunks tile each block: a stop lands on a block's end */
	S.nch = (rows + S.chunk - 1) / S.chunk;
	for (int k = 0; k < NSLOT; k++) {
		S.in_b[k] = host_buf((size_t)S.chunk * r->per * 4, &S.pin[k][0]);
		S.out_b[k] = host_buf((size_t)S.chunk * r->nout * 4, &S.pin[k][1]);
		S.st_b[k] = host_buf((size_t)S.chunk * r->nt * 4, &S.pin[k][2]);
		if (!S.in_b[k] || !S.out_b[k] || !S.st_b[k]) {
			snprintf(r->err, sizeof r->err, "out of memory");
			return -1;
		}
	}
	pthread_mutex_init(&S.mu, NULL);
	pthread_cond_init(&S.cv, NULL);
	pthread_t rd, wr;
	sigset_t stop, old; /* stop requests stay with this thread (the reader's and writer's I/O is not interrupted) */
	sigemptyset(&stop);
	sigaddset(&stop, SIGINT);
	sigaddset(&stop, SIGTERM);
	pthread_sigmask(SIG_BLOCK, &stop, &old);
	const int erd = pthread_create(&rd, NULL, stream_reader, &S);
	const int ewr = erd ? 0 : pthread_create(&wr, NULL, stream_writer, &S);
	pthread_sigmask(SIG_SETMASK, &old, NULL);
	if (erd) {
		snprintf(r->err, sizeof r->err, "cannot start the reader thread");
		return -1;
	}
	if (ewr) {
		pthread_mutex_lock(&S.mu);
		S.quit = 1;
		pthread_cond_broadcast(&S.cv);
		pthread_mutex_unlock(&S.mu);
		pthread_join(rd, NULL);
		snprintf(r->err, sizeof r->err, "cannot start the writer thread");
		return -1;
	}
	int rc = 0;
	long i = 0;
	for (; i < S.nch; i++) {
		const int k = (int)(i % NSLOT);
		pthread_mutex_lock(&S.mu);
		while (S.state[k] != 1) pthread_cond_wait(&S.cv, &S.mu);
		const long n = S.n[k];
		pthread_mutex_unlock(&S.mu);
		if (n < 0) {
			snprintf(r->err, sizeof r->err, "cannot read the rows");
			rc = -1;
			break;
		}
		if (run_block(r, S.in_b[k], n, S.out_b[k], S.st_b[k])) {
			rc = -1;
			break;
		}
		pthread_mutex_lock(&S.mu);
		S.state[k] = 2;
		pthread_cond_broadcast(&S.cv);
		pthread_mutex_unlock(&S.mu);
		block_done(r, n, block);
		if (atomic_load(&stop_sig) && (r->done % block == 0 || r->done == rows)) {
			i++;
			break; /* a stop request: this block is the last */
		}
	}
	pthread_mutex_lock(&S.mu); /* the reader stops, the writer writes the chunks computed (i of them) and stops */
	S.last = i;
	S.quit = 1;
	pthread_cond_broadcast(&S.cv);
	pthread_mutex_unlock(&S.mu);
	pthread_join(rd, NULL);
	pthread_join(wr, NULL);
	pthread_mutex_destroy(&S.mu);
	pthread_cond_destroy(&S.cv);
	for (int k = 0; k < NSLOT; k++) {
		host_buf_free(S.in_b[k], S.pin[k][0]);
		host_buf_free(S.out_b[k], S.pin[k][1]);
		host_buf_free(S.st_b[k], S.pin[k][2]);
	}
	return rc;
}

int main(int argc, char **argv)
{
	const char *model = NULL, *data = NULL, *opath = NULL, *lpath = NULL;
	int flags = 0, verbose = 0, maxrows = 16384;
	if (argc >= 2 && !strcmp(argv[1], "fxparse")) { /* the --fixed text rule, for tests (no device) */
		for (int i = 2; i < argc; i++) {
			int32_t q;
			const char *e = fx_parse(argv[i], &q);
			if (!e || *e) printf("error\n");
			else printf("%d\n", q);
		}
		return 0;
	}
	if (argc >= 2 && !strcmp(argv[1], "c")) return emit_unit(argc, argv);
	if (argc >= 2 && !strcmp(argv[1], "ir")) return print_ir(argc, argv);
	if (argc >= 2 && !strcmp(argv[1], "quantize")) return quantize(argc, argv);
	if (argc >= 2 && !strcmp(argv[1], "stream")) return stream_main(argc, argv);
	if (argc >= 2 && !strcmp(argv[1], "serve")) return serve_main(argc, argv);
	if (argc < 2 || strcmp(argv[1], "batch")) return die(USAGE, "");
	for (int i = 2; i < argc; i++) {
		if (!strcmp(argv[i], "-o") && i + 1 < argc) opath = argv[++i];
		else if (!strcmp(argv[i], "--log") && i + 1 < argc) lpath = argv[++i];
		else if (!strcmp(argv[i], "--fixed")) flags |= TG_HIP_FIXED;
		else if (!strcmp(argv[i], "--exact")) flags |= TG_HIP_EXACT;
		else if (!strcmp(argv[i], "--rows") && i + 1 < argc) maxrows = atoi(argv[++i]);
		else if (!strcmp(argv[i], "-v")) verbose = 1;
		else if (!model) model = argv[i];
		else if (!data) data = argv[i];
		else return die("unexpected argument '%s'", argv[i]);
	}
	if (!model || !data || maxrows < 1) return die(USAGE, "");
	const int fixed = (flags & TG_HIP_FIXED) != 0;
	FILE *lf = NULL;
	if (lpath && !(lf = fopen(lpath, "a"))) return die("cannot open log '%s'", lpath);
	double t0 = now_ms();
	size_t mlen;
	char lerr[1024];
	char *text = load_model(model, &mlen, lerr, sizeof lerr);
	if (!text) return die("%s", lerr);
	if (tg_hip_init(0)) return die("%s", tg_hip_error());
	tg_hip_prog *p = tg_hip_load(text, mlen, flags, maxrows);
	free(text);
	if (!p) return die("%s", tg_hip_error());
	int per, nout, nthink;
	tg_hip_info(p, &per, &nout, &nthink);
	Run run = { .p = p, .per = per, .nout = nout, .nthink = nthink, .nt = nthink ? nthink : 1, .fixed = fixed };
	char err[512];
	long rows;
	double tb = now_ms(); /* the reference's batch timer starts before the input load (src/main.c:413) */
	install_signals();    /* a stop request ends the batch after the current block */
	const char *ra = getenv("TGC_HIP_TEST_SIGTERM_AFTER_BLOCKS");
	run.raise_after = ra ? atol(ra) : 0;
	run.obin = opath && is_binary(opath);
	run.ssum = calloc((size_t)run.nt, sizeof *run.ssum);
	run.smin = calloc((size_t)run.nt, sizeof *run.smin);
	run.smax = calloc((size_t)run.nt, sizeof *run.smax);
	FILE *f = NULL;
	if (is_binary(data)) { /* raw f32 rows: checked by size, then streamed through pinned slots */
		FILE *in = fopen(data, "rb");
		long len = -1;
		if (in && !fseek(in, 0, SEEK_END)) len = ftell(in);
		if (len < 0 || fseek(in, 0, SEEK_SET)) return die("cannot read '%s'", data);
		if (len % 4 || (len / 4) % per) {
			snprintf(err, sizeof err, "'%s': %ld bytes is not a whole number of %d-float rows", data, len, per);
			return die("%s", err);
		}
		rows = len / 4 / per;
		if (!(f = opath ? fopen(opath, run.obin ? "wb" : "w") : stdout)) return die("cannot write '%s'", opath);
		run.f = f;
		if (stream_rows(&run, in, rows, maxrows)) return die("%s", run.err[0] ? run.err : tg_hip_error());
		fclose(in);
	} else {
		int rows_pinned;
		float *all = load_rows(data, per, &rows, err, sizeof err, fixed, &rows_pinned); /* validated before the output exists */
		if (!all) return die("%s", err);
		if (!(f = opath ? fopen(opath, run.obin ? "wb" : "w") : stdout)) return die("cannot write '%s'", opath);
		run.f = f;
		const long block = maxrows;
		int out_pinned, steps_pinned;
		float *out = host_buf((size_t)(rows < block ? (rows ? rows : 1) : block) * nout * sizeof *out, &out_pinned);
		int *steps = host_buf((size_t)(rows < block ? (rows ? rows : 1) : block) * run.nt * sizeof *steps, &steps_pinned);
		for (long b0 = 0; b0 < rows && !atomic_load(&stop_sig); b0 += block) {
			const long n = rows - b0 < block ? rows - b0 : block;
			if (run_block(&run, all + (size_t)b0 * per, n, out, steps)) return die("%s", tg_hip_error());
			write_block(f, run.obin, fixed, out, steps, n, nout, nthink, run.nt);
			block_done(&run, n, block);
		}
		host_buf_free(all, rows_pinned);
		host_buf_free(out, out_pinned);
		host_buf_free(steps, steps_pinned);
	}
	const long done = run.done;
	const double dev_ms = run.dev_ms;
	long *ssum = run.ssum;
	int *smin = run.smin, *smax = run.smax;
	if (opath && (ferror(f) | fclose(f))) return die("write failed '%s'", opath);
	const double ms = now_ms() - tb;
	if (verbose || lf) {
		tg_hip_stats_t st;
		tg_hip_stats(p, &st);
		char msg[512], fields[512];
		snprintf(msg, sizeof msg, "%ld row(s) in %.2f ms (%.1f us/row) on gfx950, %s executor, device %.3f ms%s", done, ms,
			 done ? 1e3 * ms / done : 0.0, st.executor ? "row-program" : "layer", dev_ms,
			 atomic_load(&stop_sig) ? " (stopped by signal)" : "");
		snprintf(fields, sizeof fields, ",\"rows\":%ld,\"threads\":1,\"sequential_rows\":0,\"ms\":%.9g,\"us_per_row\":%.9g,"
			 "\"device\":\"gfx950\",\"device_ms\":%.9g,\"load_ms\":%.9g", done, ms, done ? 1e3 * ms / done : 0.0, dev_ms, tb - t0);
		if (verbose) fprintf(stderr, "[batch] %s\n", msg);
		log_event(lf, "batch", msg, fields);
		for (int t = 0; t < nthink && done; t++) {
			snprintf(msg, sizeof msg, "think[%d] over batch: steps min %d mean %.2f max %d", t, smin[t], (double)ssum[t] / done,
				 smax[t]);
			snprintf(fields, sizeof fields, ",\"loop\":%d,\"steps_min\":%d,\"steps_mean\":%.9g,\"steps_max\":%d", t, smin[t],
				 (double)ssum[t] / done, smax[t]);
			if (verbose) fprintf(stderr, "[think] %s\n", msg);
			log_event(lf, "think", msg, fields);
		}
	}
	if (lf) fclose(lf);
	tg_hip_free(p);
	free(ssum);
	free(smin);
	free(smax);
	const int sig = atomic_load(&stop_sig);
	return sig ? 128 + sig : 0;
}
