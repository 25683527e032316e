/* tgc-hip stream and serve: the reference's connections (src/serve.c) on the
 * device batch.
 *
 *   tgc-hip stream MODEL [SRC] [-o DST] [--fixed] [--exact] [--rows N]
 *       rows in, output rows out, flushed as soon as they are computed. SRC
 *       and DST are `-` (stdin / stdout), a file, or tcp://HOST:PORT (a
 *       connection this process opens); with a tcp:// SRC and no -o, results
 *       go back over the same connection.
 *
 *   tgc-hip serve MODEL --listen [HOST:]PORT [--fixed] [--exact] [--rows N] [--window-us U]
 *       a TCP server (HOST defaults to 127.0.0.1; port 0 picks a free port,
 *       printed on stderr). A connection speaks the row protocol (rows in,
 *       one output row each, any number per connection) or HTTP/1.1, chosen
 *       by its first line: GET /health -> ok, GET / -> the model signature as
 *       JSON, POST /run -> body rows in, output rows out (text/plain).
 *
 * Rows, output rows and error lines are the reference's: values separated by
 * commas or blanks with `#` comments (blank lines give no output), outputs
 * as %.9g joined by commas with the steps of every think loop appended, a
 * malformed row answered with an `error: ...` line while the connection
 * stays usable. --fixed reads and writes Q16.16 (tg_fx_parse's rule, 6
 * decimals out), as `tgc-hip batch --fixed` does.
 *
 * The device runs batches, not rows. Every connection thread parses its rows
 * and queues them; one batcher thread owns the device program and runs
 * whatever is queued (from all connections, in arrival order, up to --rows
 * rows) as one tg_hip_batch call, then wakes the waiting connections, which
 * write their outputs in their own row order. Rows that arrive while a batch
 * runs form the next batch, so the batch size follows the load; --window-us
 * holds a batch open for up to U microseconds after its first row to gather
 * more. A connection that sends many rows at once has them read ahead and
 * queued together. Models with state updates are refused by the backend
 * (the reference serves them one row at a time in arrival order).
 *
 * SIGINT/SIGTERM stop both commands after the current rows: queued rows are
 * finished, outputs flushed, and the exit status is 128 + the signal number.
 * SIGPIPE is ignored (a peer that disconnects ends only its own connection). */
#define _GNU_SOURCE
#include "tg_hip.h"
#include "tgc_hip_cli.h"

#include <arpa/inet.h>
#include <errno.h>
#include <fcntl.h>
#include <netdb.h>
#include <netinet/in.h>
#include <poll.h>
#include <pthread.h>
#include <signal.h>
#include <stdatomic.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <strings.h>
#include <sys/socket.h>
#include <time.h>
#include <unistd.h>

/* ------------------------------------------------------------ batcher --- */

typedef struct Req {
	float *in;    /* n rows of `per` values (f32, or Q16.16 words) */
	float *out;   /* n x nout */
	int *steps;   /* n x nt */
	int n, done, failed;
	struct Req *next;
} Req;

typedef struct {
	tg_hip_prog *p;
	const char *name;
	int per, nout, nthink, nt, fixed, max_rows;
	long window_us;
	pthread_mutex_t mu;
	pthread_cond_t work, done;
	Req *head, *tail;
	int quit;
	float *in, *out; /* staging of a batch gathered from several requests */
	int *steps;
	long batches, rows;
	char err[512];
	pthread_t th;
} Batcher;

static int run_rows(Batcher *B, float *in, int n, float *out, int *steps)
{
	return B->fixed ? tg_hip_batch_fixed(B->p, (const int32_t *)in, n, (int32_t *)out, steps) : tg_hip_batch(B->p, in, n, out, steps);
}

static int queued_rows(const Batcher *B)
{
	int n = 0;
	for (const Req *r = B->head; r; r = r->next) n += r->n;
	return n;
}

static void *batcher_main(void *arg)
{
	Batcher *B = arg;
	pthread_mutex_lock(&B->mu);
	for (;;) {
		while (!B->head && !B->quit) pthread_cond_wait(&B->work, &B->mu);
		if (!B->head) break; /* stopping, nothing queued */
		if (B->window_us > 0 && !B->quit) { /* hold the batch open for more rows */
			struct timespec dl;
			clock_gettime(CLOCK_REALTIME, &dl);
			dl.tv_nsec += (B->window_us % 1000000) * 1000;
			dl.tv_sec += B->window_us / 1000000 + dl.tv_nsec / 1000000000;
			dl.tv_nsec %= 1000000000;
			while (!B->quit && queued_rows(B) < B->max_rows && pthread_cond_timedwait(&B->work, &B->mu, &dl) != ETIMEDOUT) {
			}
		}
		/* requests in arrival order up to max_rows rows (a larger request runs alone, in device passes) */
		Req *first = B->head, *last = first;
		int total = first->n;
		while (last->next && total + last->next->n <= B->max_rows) {
			last = last->next;
			total += last->n;
		}
		B->head = last->next;
		if (!B->head) B->tail = NULL;
		last->next = NULL;
		pthread_mutex_unlock(&B->mu);
		int rc;
		if (first == last) {
			rc = run_rows(B, first->in, first->n, first->out, first->steps);
		} else {
			long o = 0;
			for (Req *r = first; r; r = r->next) {
				memcpy(B->in + o * B->per, r->in, (size_t)r->n * B->per * sizeof(float));
				o += r->n;
			}
			rc = run_rows(B, B->in, total, B->out, B->steps);
			o = 0;
			for (Req *r = first; r; r = r->next) {
				memcpy(r->out, B->out + o * B->nout, (size_t)r->n * B->nout * sizeof(float));
				memcpy(r->steps, B->steps + o * B->nt, (size_t)r->n * B->nt * sizeof(int));
				o += r->n;
			}
		}
		pthread_mutex_lock(&B->mu);
		if (rc) snprintf(B->err, sizeof B->err, "%s", tg_hip_error());
		B->batches++;
		B->rows += total;
		for (Req *r = first; r; r = r->next) {
			r->done = 1;
			r->failed = rc != 0;
		}
		pthread_cond_broadcast(&B->done);
	}
	pthread_mutex_unlock(&B->mu);
	return NULL;
}

/* queue one request and wait for its batch; nonzero if the device call
 * failed, or if the batcher is stopping (requests queued before the stop
 * still run) */
static int submit(Batcher *B, Req *r)
{
	pthread_mutex_lock(&B->mu);
	if (B->quit) {
		snprintf(B->err, sizeof B->err, "the server is stopping");
		pthread_mutex_unlock(&B->mu);
		return 1;
	}
	r->next = NULL;
	r->done = r->failed = 0;
	if (B->tail) B->tail->next = r;
	else B->head = r;
	B->tail = r;
	pthread_cond_signal(&B->work);
	while (!r->done) pthread_cond_wait(&B->done, &B->mu);
	int failed = r->failed;
	pthread_mutex_unlock(&B->mu);
	return failed;
}

static int batcher_start(Batcher *B, const char *model, int flags, int max_rows, long window_us)
{
	memset(B, 0, sizeof *B);
	size_t mlen;
	char err[1024];
	char *text = load_model(model, &mlen, err, sizeof err);
	if (!text) return die("%s", err);
	if (tg_hip_init(0)) return die("%s", tg_hip_error());
	B->p = tg_hip_load(text, mlen, flags, max_rows);
	free(text);
	if (!B->p) return die("%s", tg_hip_error());
	tg_hip_info(B->p, &B->per, &B->nout, &B->nthink);
	B->name = tg_hip_model_name(B->p);
	B->nt = B->nthink ? B->nthink : 1;
	B->fixed = (flags & TG_HIP_FIXED) != 0;
	B->max_rows = max_rows;
	B->window_us = window_us;
	B->in = malloc((size_t)max_rows * B->per * sizeof(float));
	B->out = malloc((size_t)max_rows * B->nout * sizeof(float));
	B->steps = malloc((size_t)max_rows * B->nt * sizeof(int));
	if (!B->in || !B->out || !B->steps) return die("out of memory%s", "");
	pthread_mutex_init(&B->mu, NULL);
	pthread_cond_init(&B->work, NULL);
	pthread_cond_init(&B->done, NULL);
	if (pthread_create(&B->th, NULL, batcher_main, B)) return die("cannot start the batcher thread%s", "");
	return 0;
}

static void batcher_stop(Batcher *B)
{
	pthread_mutex_lock(&B->mu);
	B->quit = 1;
	pthread_cond_signal(&B->work);
	pthread_mutex_unlock(&B->mu);
	pthread_join(B->th, NULL);
	pthread_mutex_lock(&B->mu);
	tg_hip_free(B->p);
	B->p = NULL;
	pthread_mutex_unlock(&B->mu);
	free(B->in);
	free(B->out);
	free(B->steps);
}

/* -------------------------------------------------------------- rows --- */

/* A run of text lines: each becomes an output row, an `error: ...` line, or
 * nothing (blank and comment lines). Valid rows are queued together (in
 * chunks of max_rows) and the outputs written in line order. Returns the
 * lines that produced output. */
static long run_lines(Batcher *B, char **lines, int n, FILE *o)
{
	long count = 0;
	int *kind = malloc((size_t)(n ? n : 1) * sizeof *kind); /* -1 nothing, -2 error, >= 0 row index in the chunk */
	char **msg = calloc((size_t)(n ? n : 1), sizeof *msg);
	Req q = { 0 };
	q.in = malloc((size_t)(B->max_rows < n ? B->max_rows : n ? n : 1) * B->per * sizeof(float));
	q.out = malloc((size_t)(B->max_rows < n ? B->max_rows : n ? n : 1) * B->nout * sizeof(float));
	q.steps = malloc((size_t)(B->max_rows < n ? B->max_rows : n ? n : 1) * B->nt * sizeof(int));
	if (!kind || !msg || !q.in || !q.out || !q.steps) {
		fprintf(o, "error: out of memory\n");
		goto done;
	}
	for (int a = 0; a < n;) { /* one chunk: lines a..b-1 holding at most max_rows rows */
		int b = a, rows = 0;
		for (; b < n && rows < B->max_rows; b++) {
			const char *bad;
			int k = parse_row(lines[b], NULL, 0, &bad, B->fixed);
			kind[b] = -1;
			if (k == 0) continue;
			char buf[160];
			if (k < 0) {
				snprintf(buf, sizeof buf, "error: bad number near '%.20s'", bad);
			} else if (k != B->per) {
				snprintf(buf, sizeof buf, "error: row has %d values, model %s needs %d", k, B->name, B->per);
			} else {
				parse_row(lines[b], q.in + (size_t)rows * B->per, B->per, &bad, B->fixed);
				kind[b] = rows++;
				continue;
			}
			kind[b] = -2;
			msg[b] = strdup(buf);
		}
		q.n = rows;
		int failed = rows ? submit(B, &q) : 0;
		char berr[600] = "";
		if (failed) {
			pthread_mutex_lock(&B->mu);
			snprintf(berr, sizeof berr, "error: %s", B->err);
			pthread_mutex_unlock(&B->mu);
		}
		char vbuf[32];
		for (int i = a; i < b; i++) {
			if (kind[i] == -1) continue;
			count++;
			if (kind[i] == -2) {
				fprintf(o, "%s\n", msg[i]);
				continue;
			}
			if (failed) {
				fprintf(o, "%s\n", berr);
				continue;
			}
			const float *y = q.out + (size_t)kind[i] * B->nout;
			for (int j = 0; j < B->nout; j++) {
				if (B->fixed) {
					int32_t w;
					memcpy(&w, &y[j], 4);
					fx_format(w, vbuf);
					fprintf(o, "%s%s", j ? "," : "", vbuf);
				} else {
					fprintf(o, "%s%.9g", j ? "," : "", (double)y[j]);
				}
			}
			for (int t = 0; t < B->nthink; t++) fprintf(o, ",%d", q.steps[(size_t)kind[i] * B->nt + t]);
			fputc('\n', o);
		}
		a = b;
	}
done:
	for (int i = 0; i < n; i++) free(msg ? msg[i] : NULL);
	free(msg);
	free(kind);
	free(q.in);
	free(q.out);
	free(q.steps);
	return count;
}

/* ---------------------------------------------------------- line input --- */

/* the longest line (row, request or header line) a connection may send */
#define LR_MAX_LINE ((size_t)64 << 20)

typedef struct {
	int fd, eof, overflow; /* overflow: a line longer than LR_MAX_LINE arrived (its bytes are dropped, input ends) */
	char *buf;
	size_t cap, beg, end;
	size_t scan; /* buf[beg..scan) holds no '\n': a long line is searched once, not once per read */
} LR;

static void lr_init(LR *r, int fd)
{
	memset(r, 0, sizeof *r);
	r->fd = fd;
	r->cap = 1 << 16;
	r->buf = malloc(r->cap + 1);
}

/* read more input: 1 read, 0 end of input or a stop, -1 nothing available now (block = 0) */
static int lr_fill(LR *r, int block)
{
	if (!r->buf) return 0;
	if (r->scan < r->beg) r->scan = r->beg;
	if (r->beg == r->end) r->beg = r->end = r->scan = 0;
	if (r->end == r->cap) {
		if (r->beg) {
			memmove(r->buf, r->buf + r->beg, r->end - r->beg);
			r->end -= r->beg;
			r->scan -= r->beg;
			r->beg = 0;
		} else {
			char *nb = r->cap < LR_MAX_LINE ? realloc(r->buf, 2 * r->cap + 1) : NULL;
			if (!nb) { /* too long a line (or no memory for it): drop what is buffered and end the input */
				r->overflow = 1;
				r->eof = 1;
				r->beg = r->end = r->scan = 0;
				return 0;
			}
			r->buf = nb;
			r->cap *= 2;
		}
	}
	for (;;) {
		struct pollfd pf = { r->fd, POLLIN, 0 };
		int pr = poll(&pf, 1, block ? 500 : 0);
		if (pr == 0) {
			if (!block) return -1;
			if (stop_signal()) return 0;
			continue;
		}
		if (pr < 0) {
			if (errno == EINTR && !stop_signal()) continue;
			return block || errno == EINTR ? 0 : -1;
		}
		ssize_t k = read(r->fd, r->buf + r->end, r->cap - r->end);
		if (k > 0) {
			r->end += (size_t)k;
			return 1;
		}
		if (k < 0 && (errno == EINTR || errno == EAGAIN) && !stop_signal()) {
			if (!block) return -1;
			continue;
		}
		r->eof = 1;
		return 0;
	}
}

/* the next line without its line ending (valid until the next call): 1, or
 * 0 at the end of input or a stop, or -1 if no whole line is available
 * without blocking */
static int lr_line(LR *r, char **line, int block)
{
	for (;;) {
		if (!r->buf) return 0;
		if (r->scan < r->beg) r->scan = r->beg;
		char *s = r->buf + r->beg, *nl = memchr(r->buf + r->scan, '\n', r->end - r->scan);
		if (nl || (r->eof && r->end > r->beg)) {
			size_t e = nl ? (size_t)(nl - r->buf) : r->end;
			r->buf[e] = 0;
			r->beg = r->scan = nl ? e + 1 : e;
			while (e > (size_t)(s - r->buf) && r->buf[e - 1] == '\r') r->buf[--e] = 0;
			*line = s;
			return 1;
		}
		r->scan = r->end;
		if (r->eof) return 0;
		int k = lr_fill(r, block);
		if (k < 0) return -1;
		if (k == 0 && !r->eof) return 0;
	}
}

/* the row protocol from a first line on: lines already available are read
 * ahead and run as one batch; returns the lines that produced output */
static long row_session(Batcher *B, LR *in, FILE *out, char *first)
{
	long count = 0;
	int cap = 256;
	char **lines = malloc((size_t)cap * sizeof *lines);
	char *line = first;
	int rc = first ? 1 : lr_line(in, &line, 1);
	while (lines && rc == 1) {
		int n = 0;
		do {
			if (n == cap) {
				char **nl = realloc(lines, (size_t)(cap *= 2) * sizeof *lines);
				if (!nl) break;
				lines = nl;
			}
			lines[n++] = strdup(line);
		} while (n < 4 * B->max_rows && lr_line(in, &line, 0) == 1);
		count += run_lines(B, lines, n, out);
		for (int i = 0; i < n; i++) free(lines[i]);
		if (fflush(out) || stop_signal()) break; /* the peer is gone, or a stop */
		rc = lr_line(in, &line, 1);
	}
	if (in->overflow) fprintf(out, "error: line longer than %zu bytes; closing the connection\n", LR_MAX_LINE);
	free(lines);
	return count;
}

/* ------------------------------------------------------------ sockets --- */

static void split_hostport(const char *spec, char *host, size_t hn, char *port, size_t pn)
{
	const char *c = strrchr(spec, ':');
	if (!c) {
		snprintf(host, hn, "127.0.0.1");
		snprintf(port, pn, "%s", spec);
		return;
	}
	snprintf(host, hn, "%.*s", (int)(c - spec), spec);
	if (!*host) snprintf(host, hn, "127.0.0.1");
	snprintf(port, pn, "%s", c + 1);
}

static int tcp_open(const char *spec, int listening, char *err, size_t errn)
{
	char host[256], port[32];
	split_hostport(spec, host, sizeof host, port, sizeof port);
	struct addrinfo hints, *res;
	memset(&hints, 0, sizeof hints);
	hints.ai_socktype = SOCK_STREAM;
	hints.ai_flags = listening ? AI_PASSIVE : 0;
	int rc = getaddrinfo(host, port, &hints, &res);
	if (rc) {
		snprintf(err, errn, "%s%s: %s", listening ? "--listen " : "tcp://", spec, gai_strerror(rc));
		return -1;
	}
	int fd = -1, one = 1;
	for (struct addrinfo *a = res; a && fd < 0; a = a->ai_next) {
		fd = socket(a->ai_family, a->ai_socktype, a->ai_protocol);
		if (fd < 0) continue;
		if (listening) setsockopt(fd, SOL_SOCKET, SO_REUSEADDR, &one, sizeof one);
		if (listening ? (bind(fd, a->ai_addr, a->ai_addrlen) || listen(fd, 64)) : connect(fd, a->ai_addr, a->ai_addrlen)) {
			close(fd);
			fd = -1;
		}
	}
	freeaddrinfo(res);
	if (fd < 0) snprintf(err, errn, "%s%s: %s", listening ? "--listen " : "tcp://", spec, strerror(errno));
	return fd;
}

/* ------------------------------------------------------------- stream --- */

static int open_end(const char *spec, int reading, int *fd, FILE **f)
{
	char err[512];
	*fd = -1;
	*f = NULL;
	if (!spec || !strcmp(spec, "-")) {
		if (reading) *fd = 0;
		else *f = stdout;
		return 0;
	}
	if (!strncmp(spec, "tcp://", 6)) {
		int s = tcp_open(spec + 6, 0, err, sizeof err);
		if (s < 0) return die("%s", err);
		if (reading) *fd = s;
		else if (!(*f = fdopen(s, "w"))) return die("tcp://%s: cannot write", spec + 6);
		return 0;
	}
	if (reading) {
		if ((*fd = open(spec, O_RDONLY)) < 0) return die("cannot open '%s'", spec);
	} else if (!(*f = fopen(spec, "w"))) {
		return die("cannot open '%s'", spec);
	}
	return 0;
}

static int parse_common(const char *a, const char *b, int *flags, int *rows, int *used)
{
	*used = 1;
	if (!strcmp(a, "--fixed")) *flags |= TG_HIP_FIXED;
	else if (!strcmp(a, "--exact")) *flags |= TG_HIP_EXACT;
	else if (!strcmp(a, "--rows") && b) *rows = atoi(b), *used = 2;
	else return 0;
	return 1;
}

int stream_main(int argc, char **argv)
{
	const char *model = NULL, *src = NULL, *dst = NULL;
	int flags = 0, rows = 4096;
	for (int i = 2; i < argc; i++) {
		int used;
		if (!strcmp(argv[i], "-o") && i + 1 < argc) dst = argv[++i];
		else if (parse_common(argv[i], i + 1 < argc ? argv[i + 1] : NULL, &flags, &rows, &used)) i += used - 1;
		else if (!model) model = argv[i];
		else if (!src) src = argv[i];
		else return die("unexpected argument '%s'", argv[i]);
	}
	if (!model || rows < 1) return die("usage: tgc-hip stream MODEL [SRC] [-o DST] [--fixed] [--exact] [--rows N]%s", "");
	install_signals();
	Batcher B;
	if (batcher_start(&B, model, flags, rows, 0)) return 1;
	int ifd;
	FILE *ignore, *out;
	if (open_end(src, 1, &ifd, &ignore)) return 1;
	if (!dst && src && !strncmp(src, "tcp://", 6)) { /* reply over the same connection */
		if (!(out = fdopen(dup(ifd), "w"))) return die("%s: cannot write", src);
	} else {
		int ofd;
		if (open_end(dst, 0, &ofd, &out)) return 1;
	}
	LR in;
	lr_init(&in, ifd);
	row_session(&B, &in, out, NULL);
	free(in.buf);
	if (out != stdout) fclose(out);
	else fflush(out);
	if (ifd > 0) close(ifd);
	batcher_stop(&B);
	int sig = stop_signal();
	return sig ? 128 + sig : 0;
}

/* -------------------------------------------------------------- serve --- */

/* One HTTP/1.1 exchange per connection: the request head (its first line
 * already read), an optional body, one response, then the connection closes.
 * The routes, status lines, headers and bodies are the reference's wire
 * format (src/serve.c): GET /health, GET / (the signature as JSON),
 * POST /run (body rows in, output rows out), 404 for anything else, 400 for
 * a request line without a path, 413 for a body over 64 MiB. */

#define HTTP_MAX_BODY (64L << 20)

typedef struct {
	char method[8], path[256]; /* the request line's first two words (at most 7 and 255 bytes) */
	long length;               /* Content-Length (0 when absent) */
} HttpHead;

typedef struct {
	int status;
	const char *reason, *type;
	FILE *body; /* the response body, gathered before the head is written */
} HttpReply;

/* the first whitespace-separated word of s (at most cap - 1 bytes) into w; the rest after it */
static const char *word_of(const char *s, char *w, size_t cap)
{
	while (*s == ' ' || *s == '\t') s++;
	size_t n = 0;
	while (*s && *s != ' ' && *s != '\t' && *s != '\r' && *s != '\n') {
		if (n + 1 < cap) w[n++] = *s;
		s++;
	}
	w[n] = 0;
	return s;
}

static int http_head(LR *in, const char *request_line, HttpHead *h)
{
	memset(h, 0, sizeof *h);
	const char *rest = word_of(request_line, h->method, sizeof h->method);
	word_of(rest, h->path, sizeof h->path);
	char *line;
	while (lr_line(in, &line, 1) == 1 && *line) /* header lines up to the blank line */
		if (!strncasecmp(line, "content-length:", 15)) h->length = strtol(line + 15, NULL, 10);
	return h->method[0] && h->path[0];
}

static void http_send(FILE *o, const HttpReply *r, const char *body, size_t len)
{
	fprintf(o, "HTTP/1.1 %d %s\r\nContent-Type: %s\r\nContent-Length: %zu\r\nConnection: close\r\n\r\n", r->status, r->reason, r->type, len);
	fwrite(body, 1, len, o);
}

static long route_health(Batcher *B, LR *in, const HttpHead *h, HttpReply *r)
{
	(void)B, (void)in, (void)h;
	fputs("ok\n", r->body);
	return 0;
}

static long route_signature(Batcher *B, LR *in, const HttpHead *h, HttpReply *r)
{
	(void)in, (void)h;
	char sig[8192];
	r->type = "application/json";
	pthread_mutex_lock(&B->mu); /* the program stays loaded until batcher_stop, which takes this lock to free it */
	const int have = !B->quit && tg_hip_signature(B->p, sig, sizeof sig) > 0;
	pthread_mutex_unlock(&B->mu);
	if (have) fputs(sig, r->body);
	return 0;
}

/* exactly n bytes of body: what the line reader holds, then the socket */
static size_t read_body(LR *in, char *dst, size_t n)
{
	size_t got = 0;
	while (got < n) {
		if (in->end > in->beg) {
			size_t k = in->end - in->beg;
			if (k > n - got) k = n - got;
			memcpy(dst + got, in->buf + in->beg, k);
			in->beg += k, got += k;
		} else if (lr_fill(in, 1) <= 0) {
			break;
		}
	}
	return got;
}

static long route_run(Batcher *B, LR *in, const HttpHead *h, HttpReply *r)
{
	if (h->length < 0 || h->length > HTTP_MAX_BODY) {
		r->status = 413, r->reason = "Payload Too Large";
		fputs("body too large\n", r->body);
		return 0;
	}
	char *text = malloc((size_t)h->length + 1);
	if (!text) return 0;
	text[read_body(in, text, (size_t)h->length)] = 0;
	long nl = 1;
	for (const char *c = text; *c; c++) nl += *c == '\n';
	char **lines = malloc((size_t)nl * sizeof *lines);
	long rows = 0;
	if (lines) {
		int n = 0;
		for (char *c = text; *c;) { /* the body's lines, '\n'-terminated or not */
			lines[n++] = c;
			char *e = strchr(c, '\n');
			if (!e) break;
			*e = 0;
			c = e + 1;
		}
		rows = run_lines(B, lines, n, r->body);
		free(lines);
	}
	free(text);
	return rows;
}

static const struct {
	const char *method, *path;
	long (*route)(Batcher *B, LR *in, const HttpHead *h, HttpReply *r);
} ROUTES[] = {
	{ "GET", "/health", route_health },
	{ "GET", "/", route_signature },
	{ "POST", "/run", route_run },
};

static long http_exchange(Batcher *B, LR *in, FILE *o, const char *request_line)
{
	HttpHead h;
	if (!http_head(in, request_line, &h)) {
		const HttpReply bad = { 400, "Bad Request", "text/plain", NULL };
		http_send(o, &bad, "bad request\n", 12);
		return 0;
	}
	char *body = NULL;
	size_t len = 0;
	HttpReply r = { 200, "OK", "text/plain", open_memstream(&body, &len) };
	if (!r.body) return 0;
	long rows = 0;
	size_t i = 0;
	for (; i < sizeof ROUTES / sizeof ROUTES[0]; i++)
		if (!strcmp(h.method, ROUTES[i].method) && !strcmp(h.path, ROUTES[i].path)) {
			rows = ROUTES[i].route(B, in, &h, &r);
			break;
		}
	if (i == sizeof ROUTES / sizeof ROUTES[0]) {
		r.status = 404, r.reason = "Not Found";
		fputs("not found: GET /health, GET /, POST /run\n", r.body);
	}
	if (in->overflow) { /* a header line over the limit: nothing of the request is trusted */
		fclose(r.body);
		free(body);
		const HttpReply big = { 431, "Request Header Fields Too Large", "text/plain", NULL };
		http_send(o, &big, "header line too long\n", 21);
		return 0;
	}
	fclose(r.body);
	http_send(o, &r, body, len);
	free(body);
	return rows;
}

/* ------------------------------------------------------------ server --- */

/* connections served at once; more wait in the listen backlog */
#define SERVE_MAX_CONNS 256

typedef struct {
	Batcher *B;
	pthread_mutex_t mu;
	int active;      /* connection threads running */
	long rows;       /* rows answered by finished connections */
	long accepted;
} Server;

typedef struct {
	Server *S;
	int fd;
} Conn;

static void *conn_main(void *arg)
{
	Conn c = *(Conn *)arg;
	free(arg);
	FILE *out = fdopen(dup(c.fd), "w");
	LR in;
	lr_init(&in, c.fd);
	char *first;
	long rows = 0;
	if (out && lr_line(&in, &first, 1) == 1) {
		if (!strncmp(first, "GET ", 4) || !strncmp(first, "POST ", 5)) { /* HTTP, chosen by the first line */
			char *line = strdup(first);
			if (line) rows = http_exchange(c.S->B, &in, out, line);
			free(line);
		} else {
			rows = row_session(c.S->B, &in, out, first);
		}
	} else if (out && in.overflow) {
		fprintf(out, "error: line longer than %zu bytes; closing the connection\n", LR_MAX_LINE);
	}
	if (out) fclose(out);
	if (in.overflow) { /* the peer may still be sending: half-close, then read and drop for up to two seconds, so
			    * the close does not reset the connection before the peer has read our answer */
		shutdown(c.fd, SHUT_WR);
		char sink[1 << 14];
		for (int t = 0; t < 20; t++) {
			struct pollfd pf = { c.fd, POLLIN, 0 };
			if (poll(&pf, 1, 100) > 0 && read(c.fd, sink, sizeof sink) <= 0) break;
		}
	}
	free(in.buf);
	close(c.fd);
	pthread_mutex_lock(&c.S->mu);
	c.S->active--;
	c.S->rows += rows;
	pthread_mutex_unlock(&c.S->mu);
	return NULL;
}

static int server_active(Server *S)
{
	pthread_mutex_lock(&S->mu);
	const int a = S->active;
	pthread_mutex_unlock(&S->mu);
	return a;
}

/* a detached thread for connection fd (signals stay with the caller's thread) */
static void server_spawn(Server *S, int fd)
{
	Conn *c = malloc(sizeof *c);
	if (!c) {
		close(fd);
		return;
	}
	*c = (Conn){ S, fd };
	pthread_mutex_lock(&S->mu);
	S->active++;
	S->accepted++;
	pthread_mutex_unlock(&S->mu);
	sigset_t stop, old;
	sigemptyset(&stop);
	sigaddset(&stop, SIGINT);
	sigaddset(&stop, SIGTERM);
	pthread_attr_t at;
	pthread_attr_init(&at);
	pthread_attr_setdetachstate(&at, PTHREAD_CREATE_DETACHED);
	pthread_sigmask(SIG_BLOCK, &stop, &old);
	pthread_t th;
	const int rc = pthread_create(&th, &at, conn_main, c);
	pthread_sigmask(SIG_SETMASK, &old, NULL);
	pthread_attr_destroy(&at);
	if (rc) {
		close(fd);
		free(c);
		pthread_mutex_lock(&S->mu);
		S->active--;
		pthread_mutex_unlock(&S->mu);
	}
}

/* the bound address of a listening socket as HOST:PORT (port 0 picks one) */
static void bound_name(int fd, char *where, size_t n)
{
	struct sockaddr_storage sa;
	socklen_t sl = sizeof sa;
	char h[INET6_ADDRSTRLEN] = "?";
	int port = 0;
	if (getsockname(fd, (struct sockaddr *)&sa, &sl)) {
		snprintf(where, n, "?");
		return;
	}
	if (sa.ss_family == AF_INET) {
		inet_ntop(AF_INET, &((struct sockaddr_in *)&sa)->sin_addr, h, sizeof h);
		port = ntohs(((struct sockaddr_in *)&sa)->sin_port);
	} else if (sa.ss_family == AF_INET6) {
		inet_ntop(AF_INET6, &((struct sockaddr_in6 *)&sa)->sin6_addr, h, sizeof h);
		port = ntohs(((struct sockaddr_in6 *)&sa)->sin6_port);
	}
	snprintf(where, n, "%s:%d", h, port);
}

int serve_main(int argc, char **argv)
{
	const char *model = NULL, *listen_spec = NULL;
	int flags = 0, rows = 4096;
	long window = 0;
	for (int i = 2; i < argc; i++) {
		int used;
		if (!strcmp(argv[i], "--listen") && i + 1 < argc) listen_spec = argv[++i];
		else if (!strcmp(argv[i], "--window-us") && i + 1 < argc) window = atol(argv[++i]);
		else if (parse_common(argv[i], i + 1 < argc ? argv[i + 1] : NULL, &flags, &rows, &used)) i += used - 1;
		else if (!model) model = argv[i];
		else return die("unexpected argument '%s'", argv[i]);
	}
	if (!model || !listen_spec || rows < 1 || window < 0)
		return die("usage: tgc-hip serve MODEL --listen [HOST:]PORT [--fixed] [--exact] [--rows N] [--window-us U]%s", "");
	install_signals();
	char err[512];
	const int lfd = tcp_open(listen_spec, 1, err, sizeof err);
	if (lfd < 0) return die("%s", err);
	Batcher B;
	if (batcher_start(&B, model, flags, rows, window)) return 1;
	Server S = { &B, PTHREAD_MUTEX_INITIALIZER, 0, 0, 0 };
	char where[300];
	bound_name(lfd, where, sizeof where);
	fprintf(stderr, "serve: model %s on %s (%d values per row, device batches of up to %d rows); stop with SIGINT or SIGTERM\n", B.name,
		where, B.per, rows);
	while (!stop_signal()) {
		if (server_active(&S) >= SERVE_MAX_CONNS) { /* full: leave new clients in the backlog for a moment */
			const struct timespec ts = { 0, 10000000 };
			nanosleep(&ts, NULL);
			continue;
		}
		struct pollfd pf = { lfd, POLLIN, 0 };
		if (poll(&pf, 1, 500) <= 0) continue;
		const int fd = accept(lfd, NULL, NULL);
		if (fd >= 0) server_spawn(&S, fd);
	}
	close(lfd);
	for (int i = 0; i < 50 && server_active(&S); i++) { /* let open connections finish their rows */
		const struct timespec ts = { 0, 100000000 };
		nanosleep(&ts, NULL);
	}
	/* the batcher finishes what is queued and stops; a connection still open
	 * gets an error for anything it sends from now on */
	pthread_mutex_lock(&B.mu);
	const long batches = B.batches;
	pthread_mutex_unlock(&B.mu);
	batcher_stop(&B);
	pthread_mutex_lock(&S.mu);
	const long conns = S.accepted, served = S.rows;
	pthread_mutex_unlock(&S.mu);
	fprintf(stderr, "serve: stopped by signal %d after %ld connection(s), %ld row(s) in %ld device batch(es)\n", stop_signal(), conns,
		served, batches);
	return 128 + stop_signal();
}
