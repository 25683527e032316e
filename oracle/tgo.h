/* TEST INFRASTRUCTURE ONLY — the CPU parity oracle.
 *
 * A from-scratch C restatement of the reference's `tgc batch` semantics for the
 * quantized path: the TGIR reader (src/ir.c), the per-row interpreter
 * (src/vm.c) with the f32 kernels (runtime/tg_rt.h), the Q16.16 kernels
 * (runtime/tg_rtq.h) in the instruction order of the generated fixed-point
 * unit (src/cgen.c:100-314), the
 * seeded initializers (src/lower.c:661-775) and the row-parallel batch driver
 * (src/main.c:400-444, src/par.c).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker. The product (technograd_amd/)
 * never links it.
 *
 * Parity status per function is recorded in the header comment of each
 * source file ("pinned by ..." or "parity unpinned"). */
#ifndef TGO_H
#define TGO_H

#include <stddef.h>
#include <stdint.h>

#define TGO_MAXRANK 4
#define TGO_MAXARGS 3

typedef struct {
	int rank;
	int dim[TGO_MAXRANK];
} tgo_shape;

enum { TGO_PARAM, TGO_INPUT, TGO_TMP, TGO_STATE };

/* Operation codes: the subset of the reference op table (src/ops.c:7-51) that
 * the quantized batch path uses. */
enum {
	O_CONST, O_ADD, O_SUB, O_MUL, O_DIV, O_MAX, O_MIN,
	O_NEG, O_TANH, O_RELU, O_SIGMOID, O_EXP, O_SQRT, O_GELU, O_SILU, O_SOFTPLUS, O_LOG, O_SIN, O_COS, O_FLOOR, O_STEP,
	O_MATMUL, O_SOFTMAX, O_RMSNORM, O_SUM, O_MEAN, O_TRANSPOSE, O_OUTER, O_RESHAPE, O_TAKE,
	O_THINK, O_SCAN, O_COUNT
};

typedef struct {
	int kind;
	tgo_shape sh;
	int n;          /* element count */
	char *name;     /* NULL for unnamed temporaries */
	float *data;    /* params: f32 values (dequantized for quantized params, src/ir.c:507) */
	double *d64;    /* params: the same values as double, for the double-precision interpreter (vm64.c) */
	int qbits, qaxis;
	signed char *q; /* int8 codes, or int4 packed two per byte, low nibble first */
	float *qs;      /* one scale per channel */
	int32_t *fx;    /* params in Q16.16 (src/cgen.c:449-455) */
	int32_t *fqs;   /* quant scales in Q7.24 (src/cgen.c:442) */
	int index;      /* inputs: position */
	long off;       /* temporaries: arena offset (elements) */
} tgo_value;

typedef struct tgo_block tgo_block;

typedef struct {
	int op, out, na, a[TGO_MAXARGS];
	float k;                 /* const */
	int init, maxit, yield, halt, tid;
	float eps, hthr;         /* think (src/tg.h:154-170) */
	tgo_block *body;
	/* scan (src/tg.h:135-146) */
	int T, reverse, stid, nc, nx, ny;
	int *c, *cinit, *cnext, *x, *xt, *y, *ys;
} tgo_ins;

struct tgo_block {
	tgo_ins *v;
	int len, cap;
};

typedef struct {
	char *name;
	tgo_value *val;
	int nval, capval;
	int *inputs, ninputs;
	int output, nthink;
	int nupd;       /* state updates: such models are not batch-offloadable; kept to reject them */
	tgo_block top;
	long arena;     /* per-row arena in elements (each temporary has its own slot) */
	int per;        /* input floats per row */
	int nout;       /* output floats per row */
	int fixed_ready;
} tgo_module;

/* ---- public API (ctypes) ---- */
tgo_module *tgo_load(const char *text, char *err, int errn);
void tgo_free(tgo_module *m);
int tgo_info(const tgo_module *m, int *per, int *nout, int *nthink, long *arena);
int tgo_batch(const tgo_module *m, const float *rows, long nrows, float *out, int *steps, int threads);
int tgo_batch_fixed(tgo_module *m, const int32_t *rows, long nrows, int32_t *out, int *steps, int threads);
char *tgo_write(const tgo_module *m);           /* canonical TGIR text (src/ir.c:150-202); free with tgo_str_free */
void tgo_str_free(char *s);
void tgo_rand(uint32_t seed, float scale, float *out, long n);
void tgo_to_fixed_rows(const float *in, int32_t *out, long n);
int32_t tgo_to_fixed(double v, int frac);
const char *tgo_fx_format(int32_t v, char *buf);
int64_t tgo_fx_prim(int op, int64_t a, int64_t b);
extern int tgo_plant; /* test-only planted mistakes (fixed.c) */
extern int tgo_plant64; /* test-only planted mistake of the f64 interpreter (vm.c under TGO_F64) */

/* ---- internals shared between the oracle's files ---- */
int tgo_numel(const tgo_shape *s);
void tgo_matmul_dims(const tgo_shape *a, const tgo_shape *b, int *m, int *k, int *n, int *g);
int tgo_q_axis_for(const tgo_module *m, int param, const tgo_ins *in);
int tgo_qget(const signed char *q, int bits, long i);
int tgo_bcast_desc(const tgo_shape *out, const tgo_shape *a, const tgo_shape *b, int *d);
void tgo_run_row(const tgo_module *m, const float *in, float *out, int *steps, float *arena);
void tgo_run_row64(const tgo_module *m, const double *in, double *out, int *steps, double *arena);
int tgo_prepare_f64(tgo_module *m);
int tgo_batch64(tgo_module *m, const double *rows, long nrows, double *out, int *steps, int threads);
void tgo_run_row_fixed(const tgo_module *m, const int32_t *in, int32_t *out, int *steps, int32_t *arena);
int tgo_prepare_fixed(tgo_module *m);
/* matmul observer used by GPTQ calibration (restates vm_matmul_hook, src/vm.c:50, :276) */
extern void (*tgo_matmul_hook)(void *ctx, const tgo_module *m, const tgo_ins *in, const float *a, const float *b);
extern void *tgo_hook_ctx;

#endif
