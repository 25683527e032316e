/* Sanitizer harness for the backend's host parsers (CPU only, no device).
 *
 * Built by tests/cpp/sanitize.mk with AddressSanitizer and
 * UndefinedBehaviorSanitizer (errors fatal) together with the host C sources
 * of the library (tgir_read.c, tgir_write.c, tg_quant.c, tg_gptq.c,
 * tg_front.c); this file includes the driver's two sources
 * (tgc_hip_main.c, tgc_hip_serve.c) to reach their static parsers. The
 * device entry points the driver calls are a test double defined here:
 * tg_hip_load reads the model with the library's own TGIR reader and a
 * batch answers each row with a fixed function of its values, so the row
 * protocol and HTTP code run end to end without a GPU. Nothing in the
 * product links this file.
 *
 * Every mode is a seeded, bounded fuzz (xorshift64; the same seed gives the
 * same cases) that prints its case count and exits 0 when nothing fired:
 *
 *   host_fuzz tgir  SEED ITERS FILE.tgir...   mutated TGIR text through tgm_read; a model that loads is
 *                                             written (tgm_write), read back, and must write the same text
 *   host_fuzz front SEED ITERS FILE.tg...     mutated surface text through tgf_lower, written next to links
 *                                             to everything beside the seed file (imports, initializer files)
 *   host_fuzz gptq  SEED ITERS FILE.tgir...   every eligible param quantized (RTN and GPTQ, 4 and 8 bits,
 *                                             1-3 threads) with random Hessians, rank-deficient ones and
 *                                             dead inputs included, and weights scaled to extremes
 *   host_fuzz rows  SEED ITERS                random and mutated row text through parse_row (f32 and Q16.16),
 *                                             the fixed-point tokens through fx_parse, files through load_rows
 *   host_fuzz http  SEED ITERS MODEL.tgir     mutated HTTP requests and row sessions through the server's
 *                                             connection handler over a socket pair (f32 and --fixed)
 *   host_fuzz cli   SEED ITERS MODEL.tgir     `tgc-hip batch` end to end: binary rows (streamed) against the
 *                                             same rows as text, byte for byte, with random blocks and stops
 */
#define main tgc_hip_cli_main
#include "../../technograd_amd/csrc/tgc_hip_main.c"
#undef main
#include "../../technograd_amd/csrc/tgc_hip_serve.c"

#include "tg_front.h"
#include "tg_gptq.h"
#include "tgm.h"

#include <dirent.h>
#include <sys/stat.h>

/* ------------------------------------------------------ device double --- */

static char double_err[512];

struct tg_hip_prog {
	tgm_module *m;
	int fixed;
};

int tg_hip_init(int device) { return device == 0 ? 0 : -1; }

tg_hip_prog *tg_hip_load(const char *tgir, size_t len, int flags, int max_rows)
{
	if (max_rows < 1) {
		snprintf(double_err, sizeof double_err, "max_rows must be positive");
		return NULL;
	}
	tgm_module *m = tgm_read(tgir, len, double_err, sizeof double_err);
	if (!m) return NULL;
	tg_hip_prog *p = calloc(1, sizeof *p);
	p->m = m;
	p->fixed = (flags & TG_HIP_FIXED) != 0;
	return p;
}

int tg_hip_info(const tg_hip_prog *p, int *per, int *nout, int *nthink)
{
	*per = (int)p->m->per, *nout = (int)p->m->nout, *nthink = p->m->nthink;
	return 0;
}

/* output j of a row: the sum of its values times (j + 1); steps: the row's length */
int tg_hip_batch(tg_hip_prog *p, const float *rows, long nrows, float *out, int *steps)
{
	const tgm_module *m = p->m;
	for (long r = 0; r < nrows; r++) {
		double s = 0;
		for (long i = 0; i < m->per; i++) s += rows[r * m->per + i];
		for (long j = 0; j < m->nout; j++) out[r * m->nout + j] = (float)(s * (double)(j + 1));
		for (int t = 0; t < (m->nthink ? m->nthink : 1); t++) steps[r * (m->nthink ? m->nthink : 1) + t] = (int)m->per;
	}
	return 0;
}

int tg_hip_batch_fixed(tg_hip_prog *p, const int32_t *rows, long nrows, int32_t *out, int *steps)
{
	const tgm_module *m = p->m;
	for (long r = 0; r < nrows; r++) {
		uint32_t s = 0; /* wrapping sum */
		for (long i = 0; i < m->per; i++) s += (uint32_t)rows[r * m->per + i];
		for (long j = 0; j < m->nout; j++) out[r * m->nout + j] = (int32_t)(s * (uint32_t)(j + 1));
		for (int t = 0; t < (m->nthink ? m->nthink : 1); t++) steps[r * (m->nthink ? m->nthink : 1) + t] = (int)m->per;
	}
	return 0;
}

void tg_hip_free(tg_hip_prog *p)
{
	if (!p) return;
	tgm_free(p->m);
	free(p);
}

const char *tg_hip_model_name(const tg_hip_prog *p) { return p->m->name; }

int tg_hip_signature(const tg_hip_prog *p, char *json, size_t n)
{
	return snprintf(json, n, "{\"model\":\"%s\",\"inputs\":%ld,\"outputs\":%ld}\n", p->m->name, p->m->per, p->m->nout);
}

int tg_hip_stats(const tg_hip_prog *p, tg_hip_stats_t *st)
{
	(void)p;
	memset(st, 0, sizeof *st);
	return 0;
}

void *tg_hip_host_alloc(size_t bytes) { return malloc(bytes ? bytes : 1); }
int tg_hip_host_free(void *h)
{
	free(h);
	return 0;
}

const char *tg_hip_error(void) { return double_err; }
void tg_hip_str_free(char *s) { free(s); }

char *tg_hip_surface_to_tgir(const char *path)
{
	char *t = tgf_lower(path, double_err, sizeof double_err);
	return t;
}

char *tg_hip_emit_unit(const char *tgir, size_t len, int flags, const char *kernel)
{
	(void)tgir, (void)len, (void)flags, (void)kernel;
	snprintf(double_err, sizeof double_err, "no unit writer in the sanitizer harness");
	return NULL;
}

char *tg_hip_quantize_model(const char *tgir, size_t len, int bits, int gptq, const float *calib, long ncalib, int min_size,
			    int max_k, long *bytes, char *log, size_t logn)
{
	(void)tgir, (void)len, (void)bits, (void)gptq, (void)calib, (void)ncalib, (void)min_size, (void)max_k, (void)bytes;
	if (log && logn) log[0] = 0;
	snprintf(double_err, sizeof double_err, "no device quantizer in the sanitizer harness");
	return NULL;
}

/* ------------------------------------------------------------ helpers --- */

static uint64_t rng_state;

static uint64_t rnd(void)
{
	rng_state ^= rng_state << 13;
	rng_state ^= rng_state >> 7;
	rng_state ^= rng_state << 17;
	return rng_state;
}

static size_t below(size_t n) { return n ? (size_t)(rnd() % n) : 0; }

static char *read_file(const char *path, size_t *len)
{
	FILE *f = fopen(path, "rb");
	if (!f) {
		fprintf(stderr, "host_fuzz: cannot read %s\n", path);
		exit(2);
	}
	fseek(f, 0, SEEK_END);
	long n = ftell(f);
	fseek(f, 0, SEEK_SET);
	char *b = malloc((size_t)n + 1);
	if (fread(b, 1, (size_t)n, f) != (size_t)n) exit(2);
	fclose(f);
	b[n] = 0;
	*len = (size_t)n;
	return b;
}

static const char *const PIECES[] = {
	"(", ")", " ", "\n", "\t", "0", "1", "-1", "7", "127", "-128", "1e38", "-1e-45", "nan", "inf", "-inf", "0x10",
	"1.5", ".", "e", "-", "+", "#", ",", ";", "\"", "\\", "\r\n", "999999999999", "4294967296", "-2147483649",
	"f32", "quant", "param", "input", "block", "output", "think", "scan", "matmul", "reshape", "take", "softmax",
	"rmsnorm", "let", "fn", "model", "import", "=", "@", "[", "]", "{", "}", ":", "->", "\0",
};

/* one random edit of buf[0..*len) (capacity cap), from the seed `other` too */
static void mutate_once(char *buf, size_t *len, size_t cap, const char *other, size_t olen)
{
	size_t n = *len, at = below(n + 1);
	switch (rnd() % 7) {
	case 0: /* overwrite a byte */
		if (n) buf[below(n)] = (char)(rnd() & 0xff);
		break;
	case 1: { /* insert a piece */
		const char *p = PIECES[below(sizeof PIECES / sizeof PIECES[0])];
		size_t k = *p ? strlen(p) : 1;
		if (n + k > cap) break;
		memmove(buf + at + k, buf + at, n - at);
		memcpy(buf + at, p, k);
		*len = n + k;
		break;
	}
	case 2: { /* delete a range */
		size_t k = below(n - at < 64 ? n - at + 1 : 65);
		memmove(buf + at, buf + at + k, n - at - k);
		*len = n - k;
		break;
	}
	case 3: { /* duplicate a range */
		size_t k = below(n - at < 256 ? n - at + 1 : 257);
		if (n + k > cap) break;
		memmove(buf + at + k, buf + at, n - at);
		*len = n + k;
		break;
	}
	case 4: /* truncate */
		*len = at;
		break;
	case 5: { /* splice in a piece of the other seed */
		if (!olen) break;
		size_t from = below(olen), k = below(olen - from < 128 ? olen - from + 1 : 129);
		if (n + k > cap) break;
		memmove(buf + at + k, buf + at, n - at);
		memcpy(buf + at, other + from, k);
		*len = n + k;
		break;
	}
	default: { /* change a digit run to another number */
		for (size_t i = at; i < n; i++)
			if (buf[i] >= '0' && buf[i] <= '9') {
				size_t e = i;
				while (e < n && buf[e] >= '0' && buf[e] <= '9') e++;
				char num[24];
				const int nk = snprintf(num, sizeof num, "%lld", (long long)(rnd() % 3 ? rnd() % 70000 : rnd()) - (rnd() % 4 ? 0 : 1000));
				if (n - (e - i) + (size_t)nk > cap) break;
				memmove(buf + i + nk, buf + e, n - e);
				memcpy(buf + i, num, (size_t)nk);
				*len = n - (e - i) + (size_t)nk;
				break;
			}
		break;
	}
	}
}

/* a mutated copy of seed (1-8 edits), NUL-terminated; *len its length */
static char *mutant(const char *seed, size_t slen, const char *other, size_t olen, size_t *len)
{
	const size_t cap = slen + 4096;
	char *b = malloc(cap + 1);
	memcpy(b, seed, slen);
	*len = slen;
	for (int k = rnd() & 1 ? 1 : 1 + (int)below(8); k > 0; k--) mutate_once(b, len, cap, other, olen);
	b[*len] = 0;
	return b;
}

/* a failing case's input, kept where HOST_FUZZ_SAVE names (for a rerun outside the fuzz) */
static void save_case(const char *text, size_t len)
{
	const char *path = getenv("HOST_FUZZ_SAVE");
	FILE *f = path ? fopen(path, "wb") : NULL;
	if (!f) return;
	fwrite(text, 1, len, f);
	fclose(f);
	fprintf(stderr, "host_fuzz: case written to %s\n", path);
}

typedef struct {
	char **text;
	size_t *len;
	int n;
} Seeds;

static void free_seeds(Seeds s)
{
	for (int i = 0; i < s.n; i++) free(s.text[i]);
	free(s.text);
	free(s.len);
}

static Seeds load_seeds(int argc, char **argv, int first)
{
	Seeds s = { calloc((size_t)argc, sizeof(char *)), calloc((size_t)argc, sizeof(size_t)), 0 };
	for (int i = first; i < argc; i++, s.n++) s.text[s.n] = read_file(argv[i], &s.len[s.n]);
	if (!s.n) {
		fprintf(stderr, "host_fuzz: no seed files\n");
		exit(2);
	}
	return s;
}

/* --------------------------------------------------------------- tgir --- */

/* every param value and constant finite: the reader takes back what the
 * writer prints for those (an infinite value prints as `inf`, which the
 * reference's number rule, and so the reader's, takes for a symbol) */
static int finite_module(const tgm_module *m, const tgm_block *b)
{
	if (!b) {
		for (int i = 0; i < m->nval; i++)
			if (m->val[i].data)
				for (long j = 0; j < m->val[i].n; j++)
					if (!isfinite(m->val[i].data[j])) return 0;
		for (int i = 0; i < m->nval; i++)
			if (m->val[i].qs)
				for (long j = 0; j < (m->val[i].qaxis == 0 ? m->val[i].sh.dim[0] : m->val[i].sh.dim[1]); j++)
					if (!isfinite(m->val[i].qs[j])) return 0;
		b = &m->top;
	}
	for (int i = 0; i < b->len; i++) {
		const tgm_ins *in = &b->v[i];
		if (!isfinite(in->k) || !isfinite(in->eps) || (in->body && !finite_module(m, in->body))) return 0;
	}
	return 1;
}

static int fuzz_tgir(long iters, Seeds s)
{
	long loaded = 0;
	char err[512];
	for (long it = 0; it < iters; it++) {
		const int a = (int)below((size_t)s.n), b = (int)below((size_t)s.n);
		size_t len;
		char *t = it < s.n ? strdup(s.text[it]) : mutant(s.text[a], s.len[a], s.text[b], s.len[b], &len);
		if (it < s.n) len = s.len[it];
		tgm_module *m = tgm_read(t, len, err, sizeof err);
		if (m) {
			loaded++;
			char *w = finite_module(m, NULL) ? tgm_write(m) : NULL;
			if (w) { /* the canonical text reads back to a model that writes the same text */
				tgm_module *m2 = tgm_read(w, strlen(w), err, sizeof err);
				if (!m2) {
					fprintf(stderr, "host_fuzz tgir: written text does not read back (case %ld): %s\n", it, err);
					save_case(t, len);
					return 1;
				}
				char *w2 = tgm_write(m2);
				if (!w2 || strcmp(w, w2)) {
					fprintf(stderr, "host_fuzz tgir: canonical text not stable (case %ld)\n", it);
					return 1;
				}
				free(w2);
				tgm_free(m2);
				free(w);
			}
			tgm_free(m);
		}
		free(t);
	}
	printf("tgir: %ld cases, %ld loaded\n", iters, loaded);
	return 0;
}

/* -------------------------------------------------------------- front --- */

/* a fresh directory with links to every entry beside `seed` but the seed itself */
static void link_siblings(const char *dir, const char *seed)
{
	char sdir[4096];
	snprintf(sdir, sizeof sdir, "%s", seed);
	char *slash = strrchr(sdir, '/');
	if (slash) *slash = 0;
	else snprintf(sdir, sizeof sdir, ".");
	char abs_dir[4096];
	if (!realpath(sdir, abs_dir)) return;
	DIR *d = opendir(abs_dir);
	if (!d) return;
	for (struct dirent *e; (e = readdir(d));) {
		if (e->d_name[0] == '.') continue;
		char from[8192], to[8192];
		snprintf(from, sizeof from, "%s/%s", abs_dir, e->d_name);
		snprintf(to, sizeof to, "%s/%s", dir, e->d_name);
		if (symlink(from, to) && errno != EEXIST) perror("symlink");
	}
	closedir(d);
}

static int fuzz_front(long iters, Seeds s, char **paths)
{
	char tmpl[] = "/tmp/host_fuzz_front_XXXXXX";
	char *dir = mkdtemp(tmpl);
	if (!dir) return 2;
	for (int i = 0; i < s.n; i++) link_siblings(dir, paths[i]);
	char path[4096], err[1024];
	snprintf(path, sizeof path, "%s/fuzz_case.tg", dir);
	long lowered = 0, read_back = 0;
	for (long it = 0; it < iters; it++) {
		const int a = (int)below((size_t)s.n), b = (int)below((size_t)s.n);
		size_t len;
		char *t = it < s.n ? strdup(s.text[it]) : mutant(s.text[a], s.len[a], s.text[b], s.len[b], &len);
		if (it < s.n) len = s.len[it];
		FILE *f = fopen(path, "wb");
		fwrite(t, 1, len, f);
		fclose(f);
		char *ir = tgf_lower(path, err, sizeof err);
		if (ir) { /* the lowered text through the reader too (the reference's `tgc ir` writes
			   * some text its reader refuses, e.g. a think whose body yields another
			   * shape: the front end writes the same bytes, so no read-back is required) */
			lowered++;
			tgm_module *m = tgm_read(ir, strlen(ir), err, sizeof err);
			read_back += m != NULL;
			tgm_free(m);
			free(ir);
		}
		free(t);
	}
	DIR *d = opendir(dir); /* the case file and the links */
	for (struct dirent *e; d && (e = readdir(d));) {
		if (!strcmp(e->d_name, ".") || !strcmp(e->d_name, "..")) continue;
		char p[8192];
		snprintf(p, sizeof p, "%s/%s", dir, e->d_name);
		unlink(p);
	}
	if (d) closedir(d);
	rmdir(dir);
	printf("front: %ld cases, %ld lowered, %ld of those read back\n", iters, lowered, read_back);
	return 0;
}

/* --------------------------------------------------------------- gptq --- */

static double gauss(void)
{
	const double u = ((double)(rnd() >> 11) + 0.5) / 9007199254740992.0, v = (double)(rnd() >> 11) / 9007199254740992.0;
	return sqrt(-2 * log(u)) * cos(6.283185307179586 * v);
}

static int fuzz_gptq(long iters, Seeds s)
{
	char err[512], log[8192];
	long params = 0;
	for (long it = 0; it < iters; it++) {
		const int a = (int)below((size_t)s.n);
		tgm_module *m = tgm_read(s.text[a], s.len[a], err, sizeof err);
		if (!m) {
			fprintf(stderr, "host_fuzz gptq: seed %d does not read: %s\n", a, err);
			return 2;
		}
		tgq_param *q = NULL;
		const int nq = tgq_eligible(m, (int)below(3) * 64, &q);
		for (int i = 0; i < nq; i++) {
			tgm_value *v = &m->val[q[i].v];
			const double scale = (double[]){ 1.0, 1e-30, 1e30, 0.0, 3.0 }[below(5)];
			for (long j = 0; j < v->n; j++) v->data[j] = (float)(v->data[j] * scale);
			if (rnd() % 4 == 0) /* a dead channel or input */
				for (long j = 0; j < v->n; j++)
					if ((v->qaxis == 0 ? j / v->sh.dim[1] : j % v->sh.dim[1]) == 0) v->data[j] = 0;
			const int K = q[i].K, gptq = (int)(rnd() & 1);
			if (gptq && K <= 512) {
				const int nsamp = (int)below((size_t)(2 * K + 2)); /* fewer than K: rank deficient */
				q[i].H = calloc((size_t)K * K, sizeof(double));
				double *x = malloc((size_t)K * sizeof(double));
				const int dead = (int)below((size_t)K);
				for (int t = 0; t < nsamp; t++) {
					for (int k = 0; k < K; k++) x[k] = k == dead ? 0.0 : gauss();
					for (int r = 0; r < K; r++)
						for (int c = 0; c < K; c++) q[i].H[(size_t)r * K + c] += x[r] * x[c];
				}
				q[i].nsamp = nsamp;
				free(x);
			}
			log[0] = 0;
			const int bits = rnd() & 1 ? 4 : 8;
			if (tgq_quantize_param(m, &q[i], bits, gptq, 1 + (int)below(3), log, sizeof log) == 0) {
				params++;
				const int lim = bits == 8 ? 127 : 7;
				for (long j = 0; j < v->n; j++)
					if (abs(tgm_code(v, j)) > lim) {
						fprintf(stderr, "host_fuzz gptq: code out of range (case %ld)\n", it);
						return 1;
					}
			}
			free(q[i].H);
		}
		free(q);
		tgm_free(m);
	}
	printf("gptq: %ld cases, %ld params quantized\n", iters, params);
	return 0;
}

/* --------------------------------------------------------------- rows --- */

static const char *const ROW_SEEDS[] = {
	"1, 2, 3", "-0.5 1e-3\t7e+2 # comment", "0x1p3,inf,-nan", "1.000000000001,2.5e-7", "99999999999999999999",
	"100000.5 -32768.999999 32767.9999995", "1e5 1e-6 -1e10 .5 5.", "# only a comment", "", "1,,2", "1 2 x",
	"123456789012345678901234567890.123456789012345e-20", "-0 +0 0e0", "3.4028235e38 -3.4028235e39 1e-46",
};

static int fuzz_rows(long iters)
{
	const size_t ns = sizeof ROW_SEEDS / sizeof ROW_SEEDS[0];
	char tmpl[] = "/tmp/host_fuzz_rows_XXXXXX";
	char *dir = mkdtemp(tmpl);
	if (!dir) return 2;
	char tpath[4096], bpath[4096], err[512];
	snprintf(tpath, sizeof tpath, "%s/rows.txt", dir);
	snprintf(bpath, sizeof bpath, "%s/rows.bin", dir);
	long parsed = 0;
	for (long it = 0; it < iters; it++) {
		const char *sa = ROW_SEEDS[below(ns)], *sb = ROW_SEEDS[below(ns)];
		size_t len;
		char *t = mutant(sa, strlen(sa), sb, strlen(sb), &len);
		for (int fixed = 0; fixed < 2; fixed++) {
			const char *bad = NULL;
			float v[64];
			const int n = parse_row(t, v, 64, &bad, fixed);
			if (n < 0 && !(bad >= t && bad <= t + strlen(t))) {
				fprintf(stderr, "host_fuzz rows: error position outside the line (case %ld)\n", it);
				return 1;
			}
			parsed += n >= 0;
			int32_t q;
			fx_parse(t, &q);
			char buf[32];
			fx_format((int32_t)rnd(), buf);
		}
		if (it % 16 == 0) { /* whole files: text lines of the mutants, and binary of random size */
			FILE *f = fopen(tpath, "wb");
			for (int l = 0; l < 4; l++) fprintf(f, "%s\n", t);
			fclose(f);
			long rows;
			const int per = 1 + (int)below(4);
			int pinned;
			for (int fixed = 0; fixed < 2; fixed++) {
				float *all = load_rows(tpath, per, &rows, err, sizeof err, fixed, &pinned);
				if (all) host_buf_free(all, pinned);
			}
			f = fopen(bpath, "wb");
			const size_t nb = below(64);
			for (size_t i = 0; i < nb; i++) fputc((int)(rnd() & 0xff), f);
			fclose(f);
			float *all = load_rows(bpath, per, &rows, err, sizeof err, 0, &pinned);
			if (all) host_buf_free(all, pinned);
		}
		free(t);
	}
	unlink(tpath);
	unlink(bpath);
	rmdir(dir);
	printf("rows: %ld cases, %ld lines parsed\n", iters, parsed);
	return 0;
}

/* --------------------------------------------------------------- http --- */

typedef struct {
	int fd;
	const char *data;
	size_t len;
	size_t got;   /* bytes read back */
	uint64_t rng; /* the writer's own generator (threads do not share rnd's state) */
} Peer;

static void *peer_write(void *arg)
{
	Peer *p = arg;
	size_t off = 0;
	uint64_t x = p->rng | 1;
	while (off < p->len) { /* in pieces of random size, as a network would */
		x ^= x << 13, x ^= x >> 7, x ^= x << 17;
		const size_t span = p->len - off < 4096 ? p->len - off : 4096;
		size_t k = 1 + (size_t)(x % span);
		ssize_t w = write(p->fd, p->data + off, k);
		if (w <= 0) break;
		off += (size_t)w;
	}
	shutdown(p->fd, SHUT_WR);
	return NULL;
}

static void *peer_read(void *arg)
{
	Peer *p = arg;
	char buf[1 << 14];
	for (ssize_t k; (k = read(p->fd, buf, sizeof buf)) > 0;) p->got += (size_t)k;
	return NULL;
}

static const char *const HTTP_SEEDS[] = {
	"GET /health HTTP/1.1\r\nHost: x\r\n\r\n",
	"GET / HTTP/1.1\r\n\r\n",
	"POST /run HTTP/1.1\r\nContent-Length: 12\r\n\r\n1 2 3 4\n5 6\n",
	"POST /run HTTP/1.1\r\ncontent-length: -5\r\n\r\n1",
	"POST /run HTTP/1.1\r\nContent-Length: 99999999999999999999\r\n\r\n",
	"POST /run HTTP/1.1\r\nContent-Length: 40\r\n\r\n# c\n\n1,2,3,4\nbad\n1 2\n",
	"PUT /x HTTP/1.1\r\n\r\n",
	"GET\r\n\r\n",
	"1 2 3 4\n# comment\n\n5,6,7,8\n1 2\nx\n",
	"0.5 0.25 -1 100000\r\n1e-7 3 3 3",
};

typedef struct {
	Server *S;
	const char *req;
	size_t got;
	uint64_t rng;
} Client;

/* one connection of a burst: a socket pair, the server's handler on one end in
 * this thread, the request written and the answer read on the other */
static void *burst_client(void *arg)
{
	Client *c = arg;
	int sv[2];
	if (socketpair(AF_UNIX, SOCK_STREAM, 0, sv)) return NULL;
	Peer w = { sv[1], c->req, strlen(c->req), 0, c->rng }, r = { dup(sv[1]), NULL, 0, 0, 0 };
	pthread_t tw, tr;
	pthread_create(&tw, NULL, peer_write, &w);
	pthread_create(&tr, NULL, peer_read, &r);
	Conn *cn = malloc(sizeof *cn);
	*cn = (Conn){ c->S, sv[0] };
	pthread_mutex_lock(&c->S->mu);
	c->S->active++;
	pthread_mutex_unlock(&c->S->mu);
	conn_main(cn);
	pthread_join(tw, NULL);
	pthread_join(tr, NULL);
	close(sv[1]);
	close(r.fd);
	c->got = r.got;
	return NULL;
}

static int fuzz_http(long iters, const char *model)
{
	const size_t ns = sizeof HTTP_SEEDS / sizeof HTTP_SEEDS[0];
	Batcher B[2];
	for (int fx = 0; fx < 2; fx++)
		if (batcher_start(&B[fx], model, fx ? TG_HIP_FIXED : 0, 1 + fx * 7, 0)) return 2;
	Server S[2];
	for (int fx = 0; fx < 2; fx++) {
		memset(&S[fx], 0, sizeof S[fx]);
		S[fx].B = &B[fx];
		pthread_mutex_init(&S[fx].mu, NULL);
	}
	size_t answered = 0;
	for (long it = 0; it < iters; it++) {
		const char *sa = HTTP_SEEDS[below(ns)], *sb = HTTP_SEEDS[below(ns)];
		size_t len;
		char *t = it < (long)ns ? strdup(HTTP_SEEDS[it]) : mutant(sa, strlen(sa), sb, strlen(sb), &len);
		if (it < (long)ns) len = strlen(t);
		if (it % 997 == 996 || it == iters - 1) { /* a long line (2 MiB), and last one longer than a line may be */
			const size_t big = it == iters - 1 ? LR_MAX_LINE + ((size_t)1 << 20) : (size_t)2 << 20;
			char *b = malloc(big + len + 2);
			for (size_t i = 0; i < big; i++) b[i] = "0123456789 ,."[i % 14];
			b[big] = '\n';
			memcpy(b + big + 1, t, len);
			free(t);
			t = b;
			len += big + 1;
		}
		int sv[2];
		if (socketpair(AF_UNIX, SOCK_STREAM, 0, sv)) return 2;
		Peer w = { sv[1], t, len, 0, rnd() }, r = { dup(sv[1]), NULL, 0, 0, 0 };
		pthread_t tw, tr;
		pthread_create(&tw, NULL, peer_write, &w);
		pthread_create(&tr, NULL, peer_read, &r);
		Server *srv = &S[it & 1];
		Conn *c = malloc(sizeof *c);
		*c = (Conn){ srv, sv[0] };
		pthread_mutex_lock(&srv->mu);
		srv->active++;
		pthread_mutex_unlock(&srv->mu);
		conn_main(c); /* closes sv[0] */
		pthread_join(tw, NULL);
		pthread_join(tr, NULL);
		close(sv[1]);
		close(r.fd);
		answered += r.got > 0;
		free(t);
		if (it % 100 == 99) { /* a burst of 8 connections at once into one batcher */
			Client cl[8];
			pthread_t th[8];
			for (int c = 0; c < 8; c++) {
				cl[c] = (Client){ &S[0], HTTP_SEEDS[c % 2 ? 2 : 8], 0, rnd() };
				pthread_create(&th[c], NULL, burst_client, &cl[c]);
			}
			for (int c = 0; c < 8; c++) {
				pthread_join(th[c], NULL);
				if (!cl[c].got) {
					fprintf(stderr, "host_fuzz http: a burst connection got no answer (case %ld)\n", it);
					return 1;
				}
			}
		}
	}
	for (int fx = 0; fx < 2; fx++) {
		batcher_stop(&B[fx]);
		pthread_mutex_destroy(&S[fx].mu);
	}
	printf("http: %ld cases, %zu answered\n", iters, answered);
	return 0;
}

/* --------------------------------------------------------------- cli --- */

static int file_eq(const char *a, const char *b)
{
	size_t na, nb;
	char *x = read_file(a, &na), *y = read_file(b, &nb);
	const int eq = na == nb && !memcmp(x, y, na);
	free(x);
	free(y);
	return eq;
}

/* `tgc-hip batch` end to end on the device double: raw f32 rows (streamed
 * through the pinned slots by reader and writer threads) against the same
 * rows as text (read whole), byte for byte in text and binary output, f32 and
 * --fixed, blocks that do and do not divide the rows, and a stop request
 * after a block (the output holds exactly the blocks before it) */
static int check_cli(long iters, const char *model)
{
	char tmpl[] = "/tmp/host_fuzz_cli_XXXXXX";
	char *dir = mkdtemp(tmpl);
	if (!dir) return 2;
	size_t mlen;
	char *mt = read_file(model, &mlen);
	char err[512];
	tgm_module *m = tgm_read(mt, mlen, err, sizeof err);
	free(mt);
	if (!m) return 2;
	const long per = m->per, nout = m->nout;
	tgm_free(m);
	char bin[4096], txt[4096], o1[4096], o2[4096];
	snprintf(bin, sizeof bin, "%s/x.bin", dir);
	snprintf(txt, sizeof txt, "%s/x.txt", dir);
	long cases = 0;
	for (long it = 0; it < iters; it++) {
		const long rows = (long)below(40) + (it % 5 == 0 ? (long)below(3000) : 0);
		const long block = 1 + (long)below(it % 3 ? 64 : 4096);
		const int fixed = (int)(rnd() & 1), tbin = (int)(rnd() & 1);
		const long stop_after = rnd() % 4 == 0 ? 1 + (long)below(3) : 0;
		FILE *fb = fopen(bin, "wb"), *ft = fopen(txt, "w");
		for (long r = 0; r < rows; r++) {
			for (long j = 0; j < per; j++) {
				/* values exact in Q16.16 (multiples of 2^-8), so both readers agree in --fixed too */
				const float v = (float)((long)below(8192) - 4096) / 256.0f;
				fwrite(&v, 4, 1, fb);
				fprintf(ft, "%s%.9g", j ? "," : "", (double)v);
			}
			fputc('\n', ft);
		}
		fclose(fb);
		fclose(ft);
		snprintf(o1, sizeof o1, "%s/y1.%s", dir, tbin ? "bin" : "txt");
		snprintf(o2, sizeof o2, "%s/y2.%s", dir, tbin ? "bin" : "txt");
		char bs[32];
		snprintf(bs, sizeof bs, "%ld", block);
		char sa[32];
		snprintf(sa, sizeof sa, "%ld", stop_after);
		int rc[2];
		for (int v = 0; v < 2; v++) {
			char *args[] = { "tgc-hip", "batch", (char *)model, v ? txt : bin, "-o", v ? o2 : o1, "--rows", bs, fixed ? "--fixed" : NULL, NULL };
			if (stop_after) setenv("TGC_HIP_TEST_SIGTERM_AFTER_BLOCKS", sa, 1);
			atomic_store(&stop_sig, 0);
			rc[v] = tgc_hip_cli_main(fixed ? 9 : 8, args);
			unsetenv("TGC_HIP_TEST_SIGTERM_AFTER_BLOCKS");
			atomic_store(&stop_sig, 0);
		}
		signal(SIGPIPE, SIG_IGN);
		const int stopped = stop_after && rows >= stop_after * block; /* the hook raises at the end of block stop_after */
		if (rc[0] != rc[1] || rc[0] != (stopped ? 128 + SIGTERM : 0) || !file_eq(o1, o2)) {
			fprintf(stderr, "host_fuzz cli: case %ld (rows %ld block %ld fixed %d binary out %d stop %ld): rc %d %d, outputs %s\n", it, rows,
				block, fixed, tbin, stop_after, rc[0], rc[1], file_eq(o1, o2) ? "equal" : "differ");
			return 1;
		}
		if (stopped) { /* exactly the blocks before the stop */
			size_t n;
			char *y = read_file(o1, &n);
			long lines = 0;
			for (size_t i = 0; i < n; i++) lines += y[i] == '\n';
			free(y);
			const long want = stop_after * block;
			if (tbin ? n != (size_t)want * (size_t)nout * 4 : lines != want) {
				fprintf(stderr, "host_fuzz cli: case %ld stopped with the wrong amount of output\n", it);
				return 1;
			}
		}
		cases++;
	}
	unlink(bin), unlink(txt), unlink(o1), unlink(o2);
	char y1[4096], y2[4096];
	snprintf(y1, sizeof y1, "%s/y1.bin", dir), snprintf(y2, sizeof y2, "%s/y2.bin", dir), unlink(y1), unlink(y2);
	snprintf(y1, sizeof y1, "%s/y1.txt", dir), snprintf(y2, sizeof y2, "%s/y2.txt", dir), unlink(y1), unlink(y2);
	rmdir(dir);
	printf("cli: %ld cases\n", cases);
	return 0;
}

int main(int argc, char **argv)
{
	if (argc < 4) {
		fprintf(stderr, "usage: host_fuzz tgir|front|gptq|rows|http SEED ITERS [FILES...]\n");
		return 2;
	}
	rng_state = strtoull(argv[2], NULL, 10) * 0x9E3779B97F4A7C15ull + 1;
	const long iters = strtol(argv[3], NULL, 10);
	signal(SIGPIPE, SIG_IGN);
	if (!strcmp(argv[1], "tgir") || !strcmp(argv[1], "front") || !strcmp(argv[1], "gptq")) {
		Seeds s = load_seeds(argc, argv, 4);
		const int rc = argv[1][0] == 't' ? fuzz_tgir(iters, s) : argv[1][0] == 'f' ? fuzz_front(iters, s, argv + 4) : fuzz_gptq(iters, s);
		free_seeds(s);
		return rc;
	}
	if (!strcmp(argv[1], "rows")) return fuzz_rows(iters);
	if (!strcmp(argv[1], "http") && argc == 5) return fuzz_http(iters, argv[4]);
	if (!strcmp(argv[1], "cli") && argc == 5) return check_cli(iters, argv[4]);
	fprintf(stderr, "host_fuzz: unknown mode '%s'\n", argv[1]);
	return 2;
}
