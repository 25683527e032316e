/* TEST INFRASTRUCTURE ONLY — the oracle interpreter in double precision.
 *
 * vm.c compiled a second time with its value type set to double: the same
 * operations, in the same order, on the same f32 params, constants and
 * inputs, each rounded to double instead of float (libm's double functions
 * for the transcendentals). Tests use its outputs as a high-precision truth
 * for whole models, where no closed form is at hand: an f32 result of the
 * backend that fails the 1e-5 / 4 ulp comparison with the reference must be
 * no farther from this truth than the reference's own result. It is not a
 * restatement of the reference and is not compared with it. */
#define TGO_F64 1
#include "vm.c"

#include <stdlib.h>

int tgo_prepare_f64(tgo_module *m)
{
	for (int v = 0; v < m->nval; v++) {
		tgo_value *x = &m->val[v];
		if ((x->kind != TGO_PARAM && x->kind != TGO_STATE) || x->d64) continue;
		x->d64 = malloc((size_t)(x->n ? x->n : 1) * sizeof(double));
		if (!x->d64) return -1;
		for (int i = 0; i < x->n; i++) x->d64[i] = x->data[i];
	}
	return 0;
}
