/* TEST INFRASTRUCTURE ONLY — oracle batch driver and seeded initializers.
 *
 * Batch: restates `tgc batch` (src/main.c:400-444, :231-242): every row is one
 * run of the interpreter over a private arena; rows are independent for a
 * stateless model, so a row-parallel pool (src/par.c:40-50: workers take
 * chunks of rows from an atomic counter) gives results identical to one
 * thread. Outputs land at the row's own position, steps per think loop per row.
 *
 * rand(seed, scale): restates src/lower.c:661-668 (xorshift32 13/17/5) and
 * :766-775 (seed 0 => 0x9e3779b9, u = (x >> 8) / 2^24 in f32, value
 * (2u - 1) * scale in f32).
 *
 * Pinned by: tests/golden (reference-built models whose rand() params are
 * written by the reference's ir_write; this generator reproduces them bit for
 * bit), thread invariance tests (1 thread == N threads). */
#include "tgo.h"

#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>

typedef struct {
	tgo_module *m;
	const void *rows;
	long nrows;
	void *out;
	int *steps;
	int fixed;
	atomic_long next;
	long grain;
	atomic_int failed;
} Job;

static void *worker(void *arg)
{
	Job *j = arg;
	const tgo_module *m = j->m;
	int nt = m->nthink ? m->nthink : 1;
	void *arena = malloc((size_t)(m->arena ? m->arena : 1) * (j->fixed == 2 ? 8 : 4));
	int *tmp = malloc((size_t)nt * sizeof *tmp);
	if (!arena || !tmp) {
		atomic_store(&j->failed, 1);
		free(arena);
		free(tmp);
		return NULL;
	}
	for (;;) {
		long lo = atomic_fetch_add(&j->next, j->grain);
		if (lo >= j->nrows) break;
		long hi = lo + j->grain < j->nrows ? lo + j->grain : j->nrows;
		for (long r = lo; r < hi; r++) {
			int *st = j->steps ? j->steps + r * nt : tmp;
			for (int t = 0; t < nt; t++) st[t] = 0;
			if (j->fixed == 2)
				tgo_run_row64(m, (const double *)j->rows + r * m->per, (double *)j->out + r * m->nout, st, arena);
			else if (j->fixed)
				tgo_run_row_fixed(m, (const int32_t *)j->rows + r * m->per, (int32_t *)j->out + r * m->nout, st, arena);
			else
				tgo_run_row(m, (const float *)j->rows + r * m->per, (float *)j->out + r * m->nout, st, arena);
		}
	}
	free(arena);
	free(tmp);
	return NULL;
}

static int run(tgo_module *m, const void *rows, long nrows, void *out, int *steps, int threads, int fixed)
{
	if (m->nupd) return -2; /* a self-updating model runs its rows in order: not a batch workload here */
	if (threads < 1) threads = 1;
	if (threads > 256) threads = 256;
	Job j = { m, rows, nrows, out, steps, fixed, 0, 0, 0 };
	j.grain = nrows / (16L * threads);
	if (j.grain < 1) j.grain = 1;
	pthread_t th[256];
	int started = 0;
	for (int t = 1; t < threads; t++)
		if (pthread_create(&th[started], NULL, worker, &j) == 0) started++;
	worker(&j);
	for (int t = 0; t < started; t++) pthread_join(th[t], NULL);
	return atomic_load(&j.failed) ? -1 : 0;
}

int tgo_batch(const tgo_module *m, const float *rows, long nrows, float *out, int *steps, int threads)
{
	return run((tgo_module *)m, rows, nrows, out, steps, threads, 0);
}

int tgo_batch_fixed(tgo_module *m, const int32_t *rows, long nrows, int32_t *out, int *steps, int threads)
{
	if (tgo_prepare_fixed(m)) return -1;
	return run(m, rows, nrows, out, steps, threads, 1);
}

/* the double-precision interpreter (vm64.c) over double rows: a truth for tests */
int tgo_batch64(tgo_module *m, const double *rows, long nrows, double *out, int *steps, int threads)
{
	if (tgo_prepare_f64(m)) return -1;
	return run(m, rows, nrows, out, steps, threads, 2);
}

static uint32_t xorshift(uint32_t *s)
{
	uint32_t x = *s;
	x ^= x << 13;
	x ^= x >> 17;
	x ^= x << 5;
	return *s = x;
}

void tgo_rand(uint32_t seed, float scale, float *out, long n)
{
	uint32_t s = seed ? seed : 0x9e3779b9u;
	for (long i = 0; i < n; i++) {
		float u = (float)(xorshift(&s) >> 8) / 16777216.0f;
		out[i] = (2.0f * u - 1.0f) * scale;
	}
}
