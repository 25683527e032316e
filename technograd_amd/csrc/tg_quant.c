/* Host-side RTN weight quantizer of the MI355X backend: `tgc quantize
 * --method rtn` (src/quant.c:176-200 rounding and the clip search of
 * :184-200 without a Hessian, :258-316 driver) for weights too large to
 * quantize quickly in Python. Per output channel: absmax over its K weights;
 * ten clip candidates s = absmax (1 - 0.05 g) / lim, g = 0..9; each scored by
 * the squared rounding error summed in index order, in f64 with separate
 * multiply and add (this file is compiled with -ffp-contract=off); the first
 * strictly smallest wins (a channel of zeros keeps s = 1e-8 and all-zero
 * codes); codes = clamp(nearbyint(w / s), -lim, lim); scale = (float)s.
 * Channels are independent, so they are split over threads. */
#include "tg_hip.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>

typedef struct {
	const float *w;
	int rows, cols, lim, axis;
	signed char *codes;
	float *scales;
	int c0, c1; /* channels of this thread */
} QJob;

/* weight k of channel c */
static inline double wat(const QJob *j, int c, int k)
{
	return j->axis == 0 ? (double)j->w[(size_t)c * j->cols + k] : (double)j->w[(size_t)k * j->cols + c];
}

static inline double code_for(double w, double s, int lim)
{
	if (!(s > 0)) return 0.0;
	double q = nearbyint(w / s);
	return q < -lim ? -lim : q > lim ? lim : q;
}

/* channels [c0, c1) in blocks of CB: with axis 1 (channels are columns) a
 * block's K x CB weights stay in cache across the ten candidate passes */
enum { CB = 64 };

static void *qwork(void *arg)
{
	const QJob *j = arg;
	const int K = j->axis == 0 ? j->cols : j->rows;
	double amax[CB], best[CB], bs[CB], err[CB];
	for (int b0 = j->c0; b0 < j->c1; b0 += CB) {
		const int nb = j->c1 - b0 < CB ? j->c1 - b0 : CB;
		for (int u = 0; u < nb; u++) amax[u] = 0.0;
		for (int k = 0; k < K; k++)
			for (int u = 0; u < nb; u++) {
				const double a = fabs(wat(j, b0 + u, k));
				if (a > amax[u]) amax[u] = a;
			}
		for (int u = 0; u < nb; u++) {
			best[u] = INFINITY;
			bs[u] = amax[u] == 0.0 ? 1e-8 : amax[u] / j->lim;
		}
		for (int g = 0; g < 10; g++) {
			for (int u = 0; u < nb; u++) err[u] = 0.0;
			for (int k = 0; k < K; k++)
				for (int u = 0; u < nb; u++) {
					const double s = amax[u] * (1.0 - 0.05 * g) / j->lim;
					const double w = wat(j, b0 + u, k), d = w - s * code_for(w, s, j->lim);
					err[u] = err[u] + d * d;
				}
			for (int u = 0; u < nb; u++)
				if (err[u] < best[u] && amax[u] > 0.0) {
					best[u] = err[u];
					bs[u] = amax[u] * (1.0 - 0.05 * g) / j->lim;
				}
		}
		for (int k = 0; k < K; k++)
			for (int u = 0; u < nb; u++) {
				const int c = b0 + u;
				const signed char q = (signed char)code_for(wat(j, c, k), bs[u], j->lim);
				if (j->axis == 0) j->codes[(size_t)c * j->cols + k] = q;
				else j->codes[(size_t)k * j->cols + c] = q;
			}
		for (int u = 0; u < nb; u++) j->scales[b0 + u] = (float)bs[u];
	}
	return NULL;
}

int tg_hip_quantize_rtn(const float *w, int rows, int cols, int bits, int axis, signed char *codes, float *scales, int threads)
{
	if (!w || !codes || !scales || rows <= 0 || cols <= 0 || (bits != 4 && bits != 8) || (axis != 0 && axis != 1)) return -1;
	const int C = axis == 0 ? rows : cols;
	if (threads < 1) threads = 1;
	if (threads > 256) threads = 256;
	if (threads > (C + CB - 1) / CB) threads = (C + CB - 1) / CB;
	QJob jobs[256];
	pthread_t tid[256];
	int running[256] = { 0 };
	const int per = ((C + threads - 1) / threads + CB - 1) / CB * CB;
	for (int t = 0; t < threads; t++) {
		QJob *j = &jobs[t];
		j->w = w, j->rows = rows, j->cols = cols, j->lim = bits == 8 ? 127 : 7, j->axis = axis;
		j->codes = codes, j->scales = scales;
		j->c0 = t * per < C ? t * per : C;
		j->c1 = (t + 1) * per < C ? (t + 1) * per : C;
	}
	for (int t = 1; t < threads; t++)
		if (jobs[t].c0 < jobs[t].c1) running[t] = pthread_create(&tid[t], NULL, qwork, &jobs[t]) == 0;
	qwork(&jobs[0]);
	for (int t = 1; t < threads; t++) {
		if (running[t]) pthread_join(tid[t], NULL);
		else if (jobs[t].c0 < jobs[t].c1) qwork(&jobs[t]); /* a thread that could not start: do its share here */
	}
	return 0;
}
