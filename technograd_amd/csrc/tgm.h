/* Host-side model representation of the MI355X batch backend.
 *
 * A model arrives as TGIR text (the reference's canonical program format,
 * src/ir.c:1-24) and is held here as values and nested instruction blocks.
 * The device program builder (tg_hip.hip) reads this structure; nothing in it
 * depends on the reference's own structs. */
#ifndef TGM_H
#define TGM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TGM_MAXRANK 4

enum { TGM_PARAM, TGM_INPUT, TGM_TMP, TGM_STATE };

enum {
	TGM_CONST, TGM_ADD, TGM_SUB, TGM_MUL, TGM_DIV, TGM_MAX, TGM_MIN,
	TGM_NEG, TGM_TANH, TGM_RELU, TGM_SIGMOID, TGM_EXP, TGM_SQRT, TGM_GELU, TGM_SILU, TGM_SOFTPLUS, TGM_LOG,
	TGM_SIN, TGM_COS, TGM_FLOOR, TGM_STEP,
	TGM_MATMUL, TGM_SOFTMAX, TGM_RMSNORM, TGM_SUM, TGM_MEAN, TGM_TRANSPOSE, TGM_OUTER, TGM_RESHAPE, TGM_TAKE,
	TGM_THINK, TGM_SCAN, TGM_NOPS
};

typedef struct {
	int rank;
	int dim[TGM_MAXRANK];
} tgm_shape;

typedef struct {
	int kind;
	tgm_shape sh;
	long n;
	char *name;
	float *data;          /* params: f32 values (code * scale for quantized params) */
	int qbits, qaxis;     /* quantized params: 8 or 4 bits, channel axis */
	unsigned char *q;     /* codes: int8, or int4 two per byte, element i in byte i/2, low nibble first */
	float *qs;            /* one scale per channel */
	int index;            /* inputs: position in the row */
	long in_off;          /* inputs: float offset inside a row */
} tgm_value;

typedef struct tgm_block tgm_block;

typedef struct {
	int op, out, na, a[3];
	float k;
	/* think */
	int init, maxit, yield, halt, tid;
	float eps, hthr;
	tgm_block *body;
	/* scan */
	int T, reverse, stid, nc, nx, ny;
	int *c, *cinit, *cnext, *x, *xt, *y, *ys;
} tgm_ins;

struct tgm_block {
	tgm_ins *v;
	int len, cap;
};

typedef struct {
	char *name;
	tgm_value *val;
	int nval, cap;
	int *inputs, ninputs;
	int output, nthink, nupd;
	long per, nout;
	tgm_block top;
} tgm_module;

/* Parse TGIR text; NULL on error with a message in err. */
tgm_module *tgm_read(const char *text, size_t len, char *err, size_t errn);
void tgm_free(tgm_module *m);
long tgm_numel(const tgm_shape *s);
int tgm_code(const tgm_value *v, long i); /* code i (int4 sign-extended) */
/* The canonical TGIR text of a module (tgir_write.c), malloc'd; NULL for a
 * module with state updates (not recorded by the reader) or out of memory. */
char *tgm_write(const tgm_module *m);
const char *tgm_op_name(int op);

#ifdef __cplusplus
}
#endif
#endif
