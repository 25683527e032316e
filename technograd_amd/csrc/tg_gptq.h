/* Model-level quantization (tg_gptq.c): eligible params, scales and codes,
 * RTN or GPTQ with a calibration Hessian. */
#ifndef TG_GPTQ_H
#define TG_GPTQ_H

#include "tgm.h"

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
	int v, axis, C, K; /* the param, its channel axis, channels, inputs per channel */
	double *H;         /* K x K calibration Hessian (sum of x x^T over the samples), or NULL */
	long nsamp;        /* samples in H */
} tgq_param;

/* the params `tgc quantize` would quantize (src/quant.c:42-89): their count,
 * the list in *out (malloc'd), or -1 */
int tgq_eligible(const tgm_module *m, int min_size, tgq_param **out);

/* quantize one param in place (codes, scales, data = the dequantized
 * values), GPTQ when `gptq` and q->H holds samples (H is modified); a report
 * line is appended to log. 0 on success. */
int tgq_quantize_param(tgm_module *m, tgq_param *q, int bits, int gptq, int threads, char *log, size_t logn);

#ifdef __cplusplus
}
#endif

#endif
