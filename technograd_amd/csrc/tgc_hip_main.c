/* tgc-hip: `tgc batch` on the MI355X backend.
 *
 *   tgc-hip batch MODEL.tgir DATA [-o OUT] [--fixed] [--exact] [--rows N] [-v]
 *
 * Same input/output contract as the reference's batch command
 * (src/main.c:400-444, src/io.c): DATA is raw little-endian f32 when it ends in
 * .bin or .f32, otherwise text rows of numbers separated by commas or blanks
 * with `#` comments (src/io.c:23-41); every row is validated before anything
 * is computed or the output file is created; outputs are written in input
 * order, text as %.9g with the steps of every think loop appended
 * (src/io.c:79-93), binary as raw f32 without steps. Stateful models and
 * models outside the backend are refused with a message (the reference CLI
 * runs those).
 *
 * --fixed runs the model in Q16.16 (the number system of `tgc c --fixed`
 * units): inputs are converted by rounding x * 2^16 half away from zero
 * (the decimal rule of tg_fx_parse, runtime/tg_rtq.h:375-401), text outputs
 * are printed with 6 decimals (tg_fx_format, :403-418) and binary outputs are
 * the exact f32 values q / 65536. -v prints the batch summary of
 * src/main.c:155-173 on stderr. */
#include "tg_hip.h"

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static int die(const char *fmt, const char *a)
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

/* numbers of one text line; -1 on a bad token (src/io.c:25-41 rules) */
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

static float *load_rows(const char *path, int per, long *rows, char *err, size_t errn)
{
	size_t len;
	char *raw = slurp(path, &len);
	if (!raw) {
		snprintf(err, errn, "cannot read '%s'", path);
		return NULL;
	}
	float *all = NULL;
	if (is_binary(path)) {
		if (len % 4 || (len / 4) % (size_t)per) {
			snprintf(err, errn, "'%s': %zu bytes is not a whole number of %d-float rows", path, len, per);
			free(raw);
			return NULL;
		}
		*rows = (long)(len / 4 / (size_t)per);
		all = malloc(len ? len : 4);
		const unsigned char *b = (const unsigned char *)raw;
		for (size_t i = 0; i < len / 4; i++) {
			uint32_t w = (uint32_t)b[4 * i] | (uint32_t)b[4 * i + 1] << 8 | (uint32_t)b[4 * i + 2] << 16 | (uint32_t)b[4 * i + 3] << 24;
			memcpy(&all[i], &w, 4);
		}
		free(raw);
		return all;
	}
	long n = 0;
	for (int pass = 0; pass < 2; pass++) { /* pass 0 validates and counts, pass 1 parses */
		if (pass) all = malloc((size_t)(n ? n : 1) * per * sizeof *all);
		long r = 0;
		int line = 1;
		for (char *s = raw; *s; line++) {
			char *nl = strchr(s, '\n');
			if (nl) *nl = 0;
			const char *bad;
			int k = parse_row(s, NULL, 0, &bad);
			if (k < 0) {
				snprintf(err, errn, "%s:%d: bad number near '%.20s'", path, line, bad);
				free(raw);
				free(all);
				return NULL;
			}
			if (k > 0 && k != per) {
				snprintf(err, errn, "%s:%d: row has %d values, the model needs %d", path, line, k, per);
				free(raw);
				free(all);
				return NULL;
			}
			if (k > 0) {
				if (pass) parse_row(s, all + (size_t)r * per, per, &bad);
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

static void fx_format(int32_t v, char *buf) /* 6 decimals, integer arithmetic */
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

int main(int argc, char **argv)
{
	const char *model = NULL, *data = NULL, *opath = NULL;
	int flags = 0, verbose = 0, maxrows = 16384;
	if (argc < 2 || strcmp(argv[1], "batch")) return die("usage: tgc-hip batch MODEL.tgir DATA [-o OUT] [--fixed] [--exact] [--rows N] [-v]%s", "");
	for (int i = 2; i < argc; i++) {
		if (!strcmp(argv[i], "-o") && i + 1 < argc) opath = argv[++i];
		else if (!strcmp(argv[i], "--fixed")) flags |= TG_HIP_FIXED;
		else if (!strcmp(argv[i], "--exact")) flags |= TG_HIP_EXACT;
		else if (!strcmp(argv[i], "--rows") && i + 1 < argc) maxrows = atoi(argv[++i]);
		else if (!strcmp(argv[i], "-v")) verbose = 1;
		else if (!model) model = argv[i];
		else if (!data) data = argv[i];
		else return die("unexpected argument '%s'", argv[i]);
	}
	if (!model || !data) return die("usage: tgc-hip batch MODEL.tgir DATA [-o OUT] [--fixed] [--exact] [--rows N] [-v]%s", "");
	double t0 = now_ms();
	size_t mlen;
	char *text = slurp(model, &mlen);
	if (!text) return die("cannot read '%s'", model);
	if (tg_hip_init(0)) return die("%s", tg_hip_error());
	tg_hip_prog *p = tg_hip_load(text, mlen, flags, maxrows);
	free(text);
	if (!p) return die("%s", tg_hip_error());
	int per, nout, nthink;
	tg_hip_info(p, &per, &nout, &nthink);
	int nt = nthink ? nthink : 1;
	char err[512];
	long rows;
	float *all = load_rows(data, per, &rows, err, sizeof err); /* everything is validated before the output exists */
	if (!all) return die("%s", err);
	double tb = now_ms();
	float *out = malloc((size_t)(rows ? rows : 1) * nout * sizeof *out);
	int *steps = malloc((size_t)(rows ? rows : 1) * nt * sizeof *steps);
	int rc;
	if (flags & TG_HIP_FIXED) {
		int32_t *q = malloc((size_t)(rows ? rows : 1) * per * sizeof *q);
		for (long i = 0; i < rows * per; i++) {
			double s = (double)all[i] * 65536.0;
			q[i] = s >= 2147483647.0 ? INT32_MAX : s <= -2147483648.0 ? INT32_MIN : (int32_t)llround(s);
		}
		rc = tg_hip_batch_fixed(p, q, rows, (int32_t *)out, steps);
		free(q);
	} else {
		rc = tg_hip_batch(p, all, rows, out, steps);
	}
	if (rc) return die("%s", tg_hip_error());
	double tc = now_ms();
	int obin = opath && is_binary(opath);
	FILE *f = opath ? fopen(opath, obin ? "wb" : "w") : stdout;
	if (!f) return die("cannot write '%s'", opath);
	char buf[32];
	for (long r = 0; r < rows; r++) {
		const float *y = out + (size_t)r * nout;
		if (obin) {
			for (int i = 0; i < nout; i++) {
				float v = y[i];
				if (flags & TG_HIP_FIXED) {
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
			if (flags & TG_HIP_FIXED) {
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
	if (opath && (ferror(f) | fclose(f))) return die("write failed '%s'", opath);
	if (verbose) {
		tg_hip_stats_t st;
		tg_hip_stats(p, &st);
		double ms = now_ms() - tb;
		fprintf(stderr, "[batch] %ld row(s) in %.2f ms (%.3f us/row) on gfx950, %s executor, device %.3f ms, load %.1f ms, compute %.2f ms\n",
			rows, ms, rows ? 1e3 * ms / rows : 0.0, st.executor ? "row-program" : "layer", st.batch_ms, tb - t0, tc - tb);
		for (int t = 0; t < nthink && rows; t++) {
			long sum = 0;
			int mn = steps[t], mx = steps[t];
			for (long r = 0; r < rows; r++) {
				int s = steps[(size_t)r * nt + t];
				sum += s;
				mn = s < mn ? s : mn;
				mx = s > mx ? s : mx;
			}
			fprintf(stderr, "[think] think[%d] over batch: steps min %d mean %.2f max %d\n", t, mn, (double)sum / rows, mx);
		}
	}
	tg_hip_free(p);
	free(all);
	free(out);
	free(steps);
	return 0;
}
