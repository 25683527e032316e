/* Kernel launch interface shared by the program builder (tg_hip.hip) and the
 * kernel files (kern_*.hip). All launches take the program's stream. */
#ifndef TG_KERN_H
#define TG_KERN_H

#include <hip/hip_runtime.h>
#include <stdint.h>

/* A per-row operand: element i of row r is p[r * rs + i]; rs == 0 for values
 * shared by every row (params, constants). */
typedef struct {
	const float *p;
	long rs;
} tgk_opd;

/* a GEMM's activation-digit area: digits in fragment order, and per row the
 * sum of its fixed-point values, its exponent, its class (tg_qdigits.h:
 * TGQ_GRID, TGQ_REF, TGQ_SPLIT, or TGQ_CAND before a resolve) and a split
 * row's outliers (ok: input index, -1 after the last; ox: value; nout per
 * row, tgq_nout(Kp)) */
typedef struct {
	int8_t *dig;
	long long *qsum;
	int *e, *special;
	int *ok;
	float *ox;
} tgk_qdig;

/* ---- layer executor kernels (kern_layer.hip) ---- */

enum { TGK_ADD, TGK_SUB, TGK_MUL, TGK_DIV, TGK_MAX, TGK_MIN };

/* o[r, i] = a[r, ia(i)] (op) b[r, ib(i)]; ia(i) = i, 0, amap[i] or i mod aper
 * (amode 0, 1, 2, 3) */
void tgk_binary(hipStream_t s, int op, float *o, long ors, int n, tgk_opd a, int amode, const int *amap, int aper, tgk_opd b, int bmode,
		const int *bmap, int bper, int rows);
/* unary op codes are the model op codes (TGM_NEG .. TGM_STEP) */
void tgk_unary(hipStream_t s, int op, float *o, long ors, tgk_opd a, int n, int rows);

/* A fused run of elementwise instructions over rows of n elements, as an
 * accumulator machine: inputs are loaded once into registers, and each
 * instruction works on the accumulator. Kinds: TGK_EW_LOAD (acc = register a),
 * TGK_EW_SAVE (register dst = acc), TGK_EW_BIN (acc = acc op register a, op
 * one of TGK_ADD..TGK_MIN), TGK_EW_BINR (acc = register a op acc), TGK_EW_UN
 * (acc = op(acc), op a unary TGM_ op), TGK_EW_STORE (output dst = acc). Input
 * modes are those
 * of tgk_binary: 0 elementwise, 1 one scalar per row, 2 through an index map,
 * 3 whole-row repeats (element i mod in_per). Inputs of mode 0, then those of
 * mode 3 with in_per a multiple of 4 (and fewer than 2^22 repeats in a row),
 * come first; input j is loaded into register j. */
#define TGK_EW_MAXIN 6
#define TGK_EW_MAXOUT 6
#define TGK_EW_MAXINS 24
#define TGK_EW_REGS 8
enum { TGK_EW_BIN = 1, TGK_EW_UN = 2, TGK_EW_STORE = 3, TGK_EW_LOAD = 4, TGK_EW_SAVE = 5, TGK_EW_BINR = 6 };
typedef struct {
	int kind, op, dst, a, b;
} tgk_ew_ins;
typedef struct {
	const float *in[TGK_EW_MAXIN];
	long in_rs[TGK_EW_MAXIN];
	const int *in_map[TGK_EW_MAXIN];
	int in_mode[TGK_EW_MAXIN];
	int in_per[TGK_EW_MAXIN];   /* mode 3: input element i mod in_per */
	float in_inv[TGK_EW_MAXIN]; /* mode 3: 1 / in_per, for the quotient estimate */
	float *out[TGK_EW_MAXOUT];
	long out_rs[TGK_EW_MAXOUT];
	tgk_ew_ins ins[TGK_EW_MAXINS];
	int nin, nout, nins;
} tgk_ew;
void tgk_ew_run(hipStream_t s, const tgk_ew *e, int n, int rows);

/* General matmul, one thread per output, products summed in order p = 0..k-1
 * from 0.0f with separate multiply and add (the reference's order): the exact
 * path. o[r][g][i][j] = sum_p A[r][g][i][p] B[r][g][p][j]; quant 1: A is codes
 * (element g*m*k + i*k + p of the packed param) times scale[i]; quant 2: B is
 * codes (element p*n + j) times scale[j]. */
typedef struct {
	int g, m, k, n;
	tgk_opd a;
	long ag, ai, ap;
	tgk_opd b;
	long bg, bp, bj;
	float *o;
	long ors, og, oi, oj;
	int quant, bits;
	const uint8_t *codes;
	const float *scale;
	/* causal products of a prompt's attention (tiled path only; 0 elsewhere):
	 * 1: o[i][j] is needed for j <= i only, tiles wholly above the diagonal
	 * are skipped; 2: A[i][p] is an exact 0 for p > i, so a tile of rows
	 * i0 .. i0 + TS - 1 sums p = 0 .. i0 + TS - 1 only (the omitted terms add
	 * +0 to sums that are never -0) */
	int causal;
} tgk_mm;
void tgk_matmul_exact(hipStream_t s, const tgk_mm *d, int rows);

/* softmax (op TGM_SOFTMAX) or rmsnorm over `cols`-long rows, `nrow` of them per batch row */
void tgk_rowop(hipStream_t s, int op, float *o, long ors, tgk_opd a, int nrow, int cols, int rows);
/* read `bytes` at p (16-byte aligned) in `blocks` workgroups, writing nothing but (never) sink[0] */
void tgk_read(hipStream_t s, const void *p, size_t bytes, int blocks, int *sink);
/* sum or mean of the n elements of a row */
void tgk_reduce(hipStream_t s, int op, float *o, long ors, tgk_opd a, int n, int rows);
void tgk_transpose(hipStream_t s, float *o, long ors, tgk_opd a, int g, int r, int c, int rows);
void tgk_outer(hipStream_t s, float *o, long ors, tgk_opd a, int m, tgk_opd b, int n, int rows);
void tgk_take(hipStream_t s, float *o, long ors, tgk_opd w, tgk_opd idx, int cnt, int d, int h, int rows);
/* o[r*ors + ooff + i] = a[r*a.rs + aoff + i], i < w */
void tgk_copy(hipStream_t s, float *o, long ors, long ooff, tgk_opd a, long aoff, int w, int rows);

/* A whole selective scan (T steps) of the body
 *   h = exp(reshape(dt_t) * A) * h + outer(du_t, B_t); y_t = h @ C_t
 * per row: h [D][N] (carry, updated in place), dt, du [T][D], B, C [T][N],
 * A [D][N], ys [T][D]; results bit-identical to the per-instruction kernels.
 * N must be one tgk_sscan_supported() accepts. */
bool tgk_sscan_supported(int N);
/* Neighbouring instructions folded into the scan (fuse may be NULL): with
 * dux.p set, du_t = dt_t * dux_t (du unused); with gx.p set, the stacked
 * output is (y_t + gx_t * gD) * silu(gz_t) (gx, gz [T][D] per row, gD one
 * value per channel) instead of y_t. */
typedef struct {
	tgk_opd dux, gx, gz;
	const float *gD;
} tgk_sscan_fuse;
void tgk_sscan(hipStream_t s, float *h, long hrs, tgk_opd dt, tgk_opd du, tgk_opd Bq, tgk_opd Cq, tgk_opd A, float *ys, long yrs, int D,
	       int N, int T, int reverse, int rows, const tgk_sscan_fuse *fuse);

/* ---- quantized GEMM on int8 MFMA (kern_qgemm.hip) ----
 * Y = X Wq^T with X [M][K] f32 (row m at x + (m / ni) * xr + (m % ni) * xj,
 * element k at + k * xk), Wq repacked (see tgk_qweight). Exact integer
 * products of int8/int4 codes with 3 balanced int8 limbs of each
 * activation row's 24-bit fixed-point form; the dot product is rounded to f32
 * once, then multiplied by the channel scale. */
typedef struct {
	int C, K, Kp, bits;      /* channels, inputs, inputs padded to 64 */
	int Cp;                  /* channels padded to 64 */
	uint8_t *w;              /* int8: [Cp][Kp]; int4: [Cp][Kp/2] offset-binary nibbles (see kern_qgemm.hip) */
	uint8_t *wg;             /* int4 only: the large-batch GEMM's copy, [Cp/64][Kp/32][64][16] bytes, each byte two
				    channels' codes (see kern_qgemm.hip); NULL for int8 */
	float *scale;            /* [Cp] */
	uint8_t *orig;           /* original packed codes, for the exact fallback of special rows */
	int axis;                /* original layout: 0 = [C][K], 1 = [K][C] */
} tgk_qweight;

/* KV-cache decoder kernels (kern_decode.hip). Element (sequence s, KV head j,
 * position t, d) of the current layer's cache is at
 * s kv_seq + kv_layer + (j P + t) HD + d (the decoder keeps the caches
 * layer-major: [layer][sequence][KV head][position][HD] f32). */
typedef struct {
	const float *hq, *rt;    /* normed, scaled q and k lines [rows][NQ + NKV][HD], and their x @ Rot */
	const float *qkv;        /* projection output [rows][ctot] (v after q and k) */
	long ctot;
	const float *cosT, *sinT; /* [P][HD] */
	float *qr, *K, *V;        /* rotated q [rows][NQ][HD]; caches */
	long kv_seq, kv_layer;
	int T0, p0, NQ, NKV, HD, P;
} tgk_dec_rope_args;
void tgk_dec_rope(hipStream_t s, const tgk_dec_rope_args *a, int rows);
typedef struct {
	const float *qr;          /* [seqs][NQ][HD] */
	const float *K, *V;
	float *att;               /* [seqs][NQ][HD] */
	long kv_seq, kv_layer;
	int NQ, NKV, HD, P, p;    /* keys at positions 0 .. p */
	float scale;
} tgk_dec_attn_args;
/* LDS bytes of one step's attention block for n keys (at most 65536 to launch) */
size_t tgk_dec_attn_lds(int GRP, int HD, int n);
void tgk_dec_attn(hipStream_t s, const tgk_dec_attn_args *a, int seqs);
/* token-row normalization of a step or prompt chunk, fused: h += add (mode
 * 1) or h += (o_0 + ... + o_{nh-1}) in order (mode 2, the heads' output
 * projections), then out = rmsnorm(h) * g as the row-op and multiply kernels
 * compute it, and the activation digits of out for the next GEMM.
 * tgk_dec_norm, tgk_dec_hnorm and tgk_dec_silu return true when the kernel
 * they ran resolved its candidate rows itself (a step's row counts), false
 * when the GEMM must run tgk_qgemm_split first (a prompt's many lines) */
typedef struct {
	float *h;
	long hs;
	int mode;
	const float *add;
	long adds;
	const float *o;
	long ohead;
	int nh;
	const float *g;
	float *out;
	long outs;
	int D, Kp, rows;
	tgk_qdig q;
} tgk_dec_norm_args;
#define TGK_DEC_NORM_MAX 4096 /* largest D of tgk_dec_norm */
bool tgk_dec_norm(hipStream_t s, const tgk_dec_norm_args *a);
/* per-head rmsnorm * gain of the q and k heads (line (t, j) at x + t xs + j HD),
 * into out [rows][NH][HD] and the digits of its rows t NH + j */
typedef struct {
	const float *x;
	long xs;
	const float *g;
	float *out;
	int NH, HD, Kp, rows;
	tgk_qdig q;
} tgk_dec_hnorm_args;
bool tgk_dec_hnorm(hipStream_t s, const tgk_dec_hnorm_args *a);
/* out = silu(g) * u of rows [g (FF) | u (FF)] and the digits of out */
typedef struct {
	const float *gu;
	long gus;
	float *out;
	int FF, Kp, rows;
	tgk_qdig q;
} tgk_dec_silu_args;
bool tgk_dec_silu(hipStream_t s, const tgk_dec_silu_args *a);
/* out = silu(g) * u alone (the same values), for a prompt's many rows: the
 * GEMM after it makes the digits with its own many-row digit kernel */
void tgk_dec_silu_mul(hipStream_t s, const float *gu, long gus, float *out, int FF, int rows);
#define TGK_DEC_SILU_FUSED_MAX 512 /* rows below which tgk_dec_silu's one block per row makes the digits */
/* per-head output projections of `rows` token rows, all heads in one launch,
 * values equal to the digit + matrix-core path; codes int32 [NQ][HD/4][D],
 * 4 consecutive k's int8 codes per word */
size_t tgk_dec_wo_lds(int rows, int HD);
/* one head's causal softmax over a prompt chunk's scores sc [lines][T0]
 * (line L is position L % T0 of its sequence): x = s * scale + 0 and the
 * softmax on u <= t, p = 0 above the diagonal; T0 <= TGK_DEC_PROMPT_MAX */
#define TGK_DEC_PROMPT_MAX 4088 /* 4 lines of T0 + 4 floats in 64 KiB of LDS */
void tgk_dec_causal_softmax(hipStream_t s, float *sc, int T0, long nlines, float scale);
void tgk_dec_wo(hipStream_t s, const float *att, const int *codes, const float *scales, float *out, int rows, int NQ, int HD, int D);
/* pv, pi: TGK_AM_PARTS per row of workspace (each row's parts' best) */
#define TGK_AM_PARTS 64
void tgk_dec_argmax(hipStream_t s, const float *x, long xrs, int V, int rows, float *idf, int *idi, long idi_stride, float *pv, int *pi);

int tgk_qweight_pack(tgk_qweight *w, const uint8_t *codes, const float *scale, int bits, int axis, int C, int K, hipStream_t s);
/* the same from int8 codes one per element, laid out [C][K] (axis 0) */
int tgk_qweight_pack_i8(tgk_qweight *w, const int8_t *codes, const float *scale, int bits, int C, int K, hipStream_t s);
void tgk_qweight_free(tgk_qweight *w);
/* The same repacking on the device from codes and scales already in device
 * memory (codes in the param's own layout, as tgk_qweight_pack takes them),
 * into caller memory at dst of tgk_qweight_dev_bytes(bits, C, K) bytes
 * (256-byte aligned); w->orig points at the caller's codes. Nothing is
 * allocated; asynchronous on s. Not freed with tgk_qweight_free. */
size_t tgk_qweight_dev_bytes(int bits, int C, int K);
int tgk_qweight_pack_dev(tgk_qweight *w, void *dst, const uint8_t *codes, const float *scale, int bits, int axis, int C, int K,
			 hipStream_t s);

/* Output segments of a merged GEMM (several weights that read the same
 * activations, concatenated along C): columns seg_c0[s] .. seg_c0[s + 1] - 1
 * go to segment s, column c as column c - seg_c0[s] of an output with base
 * seg_o[s], batch-row stride seg_orr[s], inner-row stride seg_oj[s] and the
 * common channel stride oc. nseg <= 1: one output (o, orr, oc, oj). */
#define TGK_QSEG 32
/* One instruction of a GEMM epilogue chain: TGK_EW_UN (v = op(v), op a TGM_
 * unary op), TGK_EW_BIN (v = v op x) or TGK_EW_BINR (v = x op v), op one of
 * TGK_ADD..TGK_MIN, with x read at mode 0: x[r xr + j oj + c oc] (a value of
 * the output's shape, the output's in-row layout), 1: x[r xr] (one value),
 * 3: x[r xr + c] (one value per channel; channel stride 1). */
#define TGK_EPI_MAX 4
typedef struct {
	int kind, op, mode;
	const float *x;
	long xr;
} tgk_epi;
typedef struct {
	const tgk_qweight *w;
	const float *x;
	long xr, xj, xk;        /* activation strides: batch row, inner row, k */
	int ni;                 /* inner rows per batch row (m = r * ni + j) */
	float *o;
	long orr, oc, oj;       /* output strides: batch row, channel, inner row */
	int M;                  /* rows of X = batch rows * ni */
	int nseg;
	int seg_c0[TGK_QSEG + 1];
	float *seg_o[TGK_QSEG];
	long seg_orr[TGK_QSEG], seg_oj[TGK_QSEG];
	/* The instructions after the product that only read its chain of results,
	 * in order: output (r, j, c) goes through epi[0], epi[1], ... (one output
	 * only: nseg <= 1); applied in the large-batch kernel's epilogue, or by
	 * tgk_qgemm_chain. */
	int nepi;
	tgk_epi epi[TGK_EPI_MAX];
	/* TGM_RMSNORM or TGM_SOFTMAX over each output line's C channels (channel
	 * stride 1), after the chain; 0: none. Applied inside the product's kernel
	 * when one workgroup holds whole lines, else by the caller (tgk_rowop). */
	int rowop;
} tgk_qgemm_args;

/* Products over at most this many inputs take the reference's sequential
 * loop for every row, bit for bit (no digits: tgk_qgemm_digits and
 * tgk_qgemm_split launch nothing for them) */
#define TGK_REFLOOP_K 32
/* scratch: bytes needed for M rows of K inputs */
/* One row of int4 weights (M = 1, unit-stride 16-byte-aligned row, K a
 * multiple of 16, K <= 8192): tgk_qgemm_fused computes the digits inside
 * the product's own kernel (and leaves them in the scratch like
 * tgk_qgemm_digits); other cases fall back to digits + product. */
bool tgk_qgemm_fusable(const tgk_qgemm_args *a);
int tgk_qgemm_fused(hipStream_t s, const tgk_qgemm_args *a, void *scratch);
size_t tgk_qgemm_scratch(int M, int Kp);
int tgk_qgemm(hipStream_t s, const tgk_qgemm_args *a, void *scratch);
/* the digit area tgk_qgemm uses in `scratch` for M rows of Kp inputs, for
 * kernels that write a GEMM's activation digits themselves (tg_qdigits.h)
 * before tgk_qgemm_mfma */
tgk_qdig tgk_qgemm_digit_area(void *scratch, int M, int Kp);
/* the two launches of tgk_qgemm: activation digits, then the MFMA kernel.
 * tgk_qgemm, tgk_qgemm_fused and tgk_qgemm_mfma return what the product's
 * kernel applied besides the products: TGK_DID_CHAIN (a->epi) and
 * TGK_DID_ROWOP (a->rowop); the caller applies the rest over the output
 * (tgk_qgemm_chain, then tgk_rowop). */
#define TGK_DID_CHAIN 1
#define TGK_DID_ROWOP 2
void tgk_qgemm_chain(hipStream_t s, const tgk_qgemm_args *a);
void tgk_qgemm_digits(hipStream_t s, const tgk_qgemm_args *a, void *scratch);
/* the resolve of candidate rows (tg_qdigits.h) over digits already in the
 * scratch, at every batch size: each keeps its grid, is split, or takes the
 * reference's loop (tgk_qgemm_digits runs it itself; producers that write
 * the digits of a materialised activation in their own kernels call it
 * before the GEMM) */
void tgk_qgemm_split(hipStream_t s, const tgk_qgemm_args *a, void *scratch);
int tgk_qgemm_mfma(hipStream_t s, const tgk_qgemm_args *a, void *scratch);

/* ---- row-program interpreter (kern_rowprog.hip) ---- */

/* One instruction of a row program (one lane runs one batch row through the
 * whole program). Operand references: ref >= 0 is an arena slot (element
 * ref + i of the lane's arena), ref < 0 is the pool word -ref - 1 + i
 * (params and constants, shared by all lanes). */
enum {
	RP_CONST, RP_BIN, RP_UN, RP_MM, RP_ROW, RP_RED, RP_TRANS, RP_OUTER, RP_COPY, RP_TAKE,
	RP_THINK, RP_THINK_END, RP_SCAN, RP_SCAN_STEP, RP_SCAN_END, RP_NOP
};

typedef struct {
	int kind, op, out, a, b, n;
	int p[10];
} rp_ins;

typedef struct {
	const rp_ins *prog;
	int nins;
	const float *pool;      /* f32 params/constants, or Q16.16 words when fixed */
	const int *imap;        /* broadcast maps referenced by RP_BIN */
	const uint8_t *codes;   /* quantized params (packed as in the model) */
	const float *fscale;    /* f32 scales */
	const int *qscale;      /* Q7.24 scales */
	float *arena;           /* [arena][R] */
	long arena_n, R;
	const float *in;        /* [rows][per] */
	int per, in_slot;
	float *out;             /* [rows][nout] */
	int nout, out_ref;
	int *steps;             /* [rows][nthink] */
	int nthink;
	int rows;
	int fixed;
	/* calibration capture (f32 programs): an RP_MM with p[8] = c + 1 appends
	 * its left operand's rows (p[9] = 1) or right operand's columns (p[9] = 0)
	 * to capture c: row r's samples at cap + cap_base[c] + (r cap_rows[c] +
	 * count) cap_k[c], count in cap_count[c * rows + r] */
	float *cap;
	const long *cap_base;
	const int *cap_k, *cap_rows;
	int *cap_count;
} rp_args;

void tgk_rowprog(hipStream_t s, const rp_args *a);
/* H[r][c] = sum over the rows in order, then each row's samples in order, of
 * x_r x_c in f64 (the order of the reference's hook): capture c of a pass */
void tgk_hessian(hipStream_t s, const float *cap, const int *count, long row_cap, int K, int rows, double *H);

#endif
