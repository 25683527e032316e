/* tg_hip: MI355X (gfx950) batch backend for Technograd's quantized `tgc batch`.
 *
 * A plain C ABI: no C++ or framework types, caller-owned host buffers, int
 * status codes (0 ok, < 0 error) with the message in tg_hip_error(). The
 * library never exits the process and never prints.
 *
 * Reference seams this replaces (file:line in the reference tree):
 *   tg_hip_load        the per-row interpreter setup `load_module` + `plan`
 *                      (src/util.c:335-369, src/plan.c:154-224): the model is
 *                      handed over as canonical TGIR text (what `ir_write`,
 *                      src/ir.c:150-202, writes for a loaded Module), and its
 *                      arena becomes one device allocation.
 *   tg_hip_batch       the block loop of `tgc batch` (src/main.c:431-441):
 *                      par_for(batch_rows) -> vm_run_into per row
 *                      (src/main.c:231-242, src/vm.c:475-481), for stateless
 *                      models (m->nupd == 0, src/main.c:435).
 *   tg_hip_batch_fixed the same over Q16.16 integers, with the kernels of a
 *                      `tgc c --fixed` unit (runtime/tg_rtq.h, src/cgen.c:100-314).
 *   tg_hip_matmul_q    one quantized matmul with tg_matmul_qa / tg_matmul_qb's
 *                      arguments (runtime/tg_rt.h:132-151), the per-instruction
 *                      dispatch point src/vm.c:277-281.
 *
 * Numerics: integer and Q16.16 results are bit-exact with the reference. f32
 * results are bit-exact except for transcendentals (device libm) and, on the
 * default path, quantized matmuls, which use int8 matrix cores with exact
 * integer products on a 24-bit grid of each row and round the dot product
 * once. Those are closer to the exact product than the reference's
 * sequential sum, but not within 1e-5 relative of the reference's value on
 * every output: at K = 4096 about 2-4 % of outputs differ from it by more
 * (each within 4 units of 2^-24 sum |s w x| of the exact product).
 * TG_HIP_EXACT selects the reference's sequential f32 order, bit for bit. A
 * row's outputs never depend on the batch it comes in. */
#ifndef TG_HIP_H
#define TG_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct tg_hip_prog tg_hip_prog;

/* tg_hip_load flags */
#define TG_HIP_FIXED   1  /* run in Q16.16 (the `--fixed` number system) */
#define TG_HIP_EXACT   2  /* quantized matmuls in the reference's sequential f32 order */
#define TG_HIP_ROWPROG 4  /* force the one-lane-per-row executor for any model */
#define TG_HIP_TIMING  8  /* time every kernel with HIP events (tg_hip_stats) */
#define TG_HIP_INTERP  16 /* row programs: run the interpreter instead of compiling the model */

typedef struct {
	int executor;        /* 0: layer executor, 1: row-program executor */
	int rows;            /* rows of the last batch */
	double batch_ms;     /* device time from the first tg_hip_batch_device call after a
	                        tg_hip_sync to the end of the last one (HIP events);
	                        for tg_hip_batch, the last call */
	double qgemm_ms;     /* time in quantized-matmul kernels (TG_HIP_TIMING) */
	long qgemm_calls;
	double digits_ms;    /* time in activation-digit kernels (TG_HIP_TIMING) */
	double other_ms;     /* time in the remaining kernels (TG_HIP_TIMING) */
	double weight_bytes; /* packed quantized weight bytes the program reads per pass */
	double macs;         /* multiply-adds of quantized matmuls per row */
	long arena_bytes;    /* device arena of the program at its row capacity */
	int rowprog_jit;     /* row program: 1 when compiled for the model (hipRTC), 0 when interpreted */
	long rowprog_hoisted; /* instructions the compiled row program runs once in front of their think loop */
	int epilogue_ins;    /* layer program: instructions after quantized products that their GEMMs apply in
	                        their epilogues (elementwise chains, softmax / rmsnorm over the channels) */
	int scan_folded_ins; /* layer program: instructions around fused selective scans that the scans' kernels
	                        apply (the du product before a scan, the gate after it) */
} tg_hip_stats_t;

/* Select the device (ordinal) for subsequent calls; 0 on success. */
int tg_hip_init(int device);

/* Build a device program from TGIR text. max_rows bounds the rows of one
 * device pass (larger batches run in passes). Returns NULL when the model is
 * outside what the backend runs (state updates, unsupported ops) or on a
 * device error; the caller then keeps the CPU interpreter. */
tg_hip_prog *tg_hip_load(const char *tgir, size_t len, int flags, int max_rows);

/* Row layout: floats per input row, per output row, think loops (steps per row). */
int tg_hip_info(const tg_hip_prog *p, int *per, int *nout, int *nthink);

/* Host buffers: rows [nrows][per] -> out [nrows][nout], steps [nrows][max(nthink,1)]
 * (steps may be NULL). Synchronous. */
int tg_hip_batch(tg_hip_prog *p, const float *rows, long nrows, float *out, int *steps);
int tg_hip_batch_fixed(tg_hip_prog *p, const int32_t *rows, long nrows, int32_t *out, int *steps);

/* Device buffers (from tg_hip_dev_alloc), nrows <= max_rows. Asynchronous on
 * the program's stream; tg_hip_sync waits. */
int tg_hip_batch_device(tg_hip_prog *p, const void *d_rows, long nrows, void *d_out, int *d_steps);
int tg_hip_sync(tg_hip_prog *p);

/* Launch on `stream` (a hipStream_t of the caller's, e.g. PyTorch's current
 * stream) instead of the program's own; NULL restores the program's stream.
 * Work already queued on the previous stream is waited for first. No
 * counterpart in the reference (its interpreter has no streams): for callers
 * that order the backend's work with their own. */
int tg_hip_set_stream(tg_hip_prog *p, void *stream);
/* The hipStream_t the program launches on (to order other work after it). */
void *tg_hip_get_stream(const tg_hip_prog *p);

/* One quantized matmul with the reference kernel's arguments, host buffers:
 * axis 0: o[m,n] = diag(s) Q[m,k] @ b[k,n]  (tg_matmul_qa)
 * axis 1: o[m,n] = b[m,k] @ Q[k,n] diag(s)  (tg_matmul_qb; b is the left operand) */
int tg_hip_matmul_q(float *o, const signed char *q, int bits, const float *s, const float *b, int m, int k, int n, int axis,
		    int flags);
/* tg_matmul_qa and tg_matmul_qb (runtime/tg_rt.h:132, :143) with their exact
 * argument lists, for a call site that swaps the function name only
 * (src/vm.c:277-281): tg_hip_matmul_q on axis 0 and 1. 0 on success. */
int tg_hip_matmul_qa(float *o, const signed char *q, int bits, const float *s, const float *b, int m, int k, int n);
int tg_hip_matmul_qb(float *o, const float *a, const signed char *q, int bits, const float *s, int m, int k, int n);

/* tg_hip_matmul_q's matrix-core path without any device allocation. No
 * counterpart in the reference: for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Device buffers: d_q codes and d_s scales in the reference layout and meaning
 * of tg_hip_matmul_q, d_b the activations, d_o the output (caller-owned).
 * Asynchronous on `stream` (a hipStream_t; NULL: the null stream). Packed
 * weights and activation digits go to a fixed device array of
 * TG_HIP_NOALLOC_SCRATCH bytes that the library holds on every GPU it runs on
 * until the process ends. With Cp = ceil(C/256)*256, Kp = ceil(K/64)*64 and
 * Mp = ceil(M/128)*128 (C channels, K inputs, M activation rows), a call
 * needs r(Cp*Kp*bits/8) bytes of packed weights, twice that for int4 (a
 * second copy in channel pairs), plus r(4*Cp) of scales, plus
 * Mp*(3*Kp + 16 + 8*min(64, Kp/16)) + 256 bytes of digits and row data
 * (r: rounded up to 256). Config 2's 4096 x 4096 int4 layer fits at up to
 * 6528 activation rows; larger calls return -2 with the sizes in
 * tg_hip_error(). Every call on a GPU uses that GPU's one array: calls that
 * overlap on one GPU (other streams, other threads) race and must be
 * serialised by the caller. 0 on success. */
#define TG_HIP_NOALLOC_SCRATCH (96u << 20)
int tg_hip_matmul_q_noalloc(float *d_o, const signed char *d_q, int bits, const float *d_s, const float *d_b, int m, int k, int n,
			    int axis, void *stream);

/* The model's row program as a freestanding HIP translation unit (weights as
 * literals, values in registers, one lane per row): the counterpart of
 * `tgc c MODEL [--fixed] -o unit.c` (src/cgen.c:458-520, unit ABI
 * docs/SPEC.md:208-221) for the device. The unit defines
 *   extern "C" __global__ void KERNEL(const T *in, T *out, int *steps, int rows)
 *   extern "C" int KERNEL_batch(const void *d_in, int rows, void *d_out, int *d_steps, hipStream_t st)
 * with T = int32 Q16.16 words under TG_HIP_FIXED, else float; device buffers
 * [rows][per] in, [rows][nout] out, [rows][nthink] steps (or NULL). It is the
 * kernel tg_hip_load compiles for such a model. Needs no GPU. `kernel` NULL:
 * tg_<model>_rows. NULL with tg_hip_error() for models the unit form does not
 * take (scans, gathers, state updates, very large rows). Free with
 * tg_hip_str_free. */
char *tg_hip_emit_unit(const char *tgir, size_t len, int flags, const char *kernel);
void tg_hip_str_free(char *s);

/* The program's model name, and its signature as the JSON object the
 * reference's `tgc serve` answers `GET /` with (src/serve.c:320-332: model,
 * inputs with their types, output type, values per row, think loops,
 * stateful) followed by a newline; returns the JSON length, or -1 (text
 * truncated to n - 1 bytes when longer). */
const char *tg_hip_model_name(const tg_hip_prog *p);
int tg_hip_signature(const tg_hip_prog *p, char *json, size_t n);

/* `tgc quantize` (src/quant.c:318-384) on the backend: the model (TGIR) with
 * its eligible params quantized to int`bits` per channel, as canonical TGIR
 * text (free with tg_hip_str_free). RTN, or with `gptq` GPTQ over a
 * calibration Hessian: the f32 model runs over the `ncalib` calibration rows
 * ([ncalib][per] f32) on the device, capturing each weight's other matmul
 * operand as the reference's hook does (src/quant.c:92-117), and the device
 * sums H = sum x x^T in the reference's order (the same f64 values). The
 * reference computes Hessians only for K <= 2048 (src/quant.c:346): with
 * max_k = 2048 the output is the reference's; max_k <= 0 gives every
 * eligible weight its Hessian (larger K diverges from the reference by
 * design). With calibration rows the log also reports the output change on
 * them (device runs of both models). RTN without calibration rows needs no
 * GPU. `log` receives the report lines; bytes (may be NULL) the params' size
 * before and after, as the reference reports it. NULL with tg_hip_error()
 * on failure. */
char *tg_hip_quantize_model(const char *tgir, size_t len, int bits, int gptq, const float *calib, long ncalib, int min_size, int max_k,
			    long *bytes, char *log, size_t logn);

/* The surface model file at `path` (.tg, with its imports and initializer
 * files) lowered to canonical TGIR text: the bytes `tgc ir MODEL.tg` prints
 * (src/main.c:373-375 over src/util.c:335-369: surface_load, lower, ir_write).
 * The result is what tg_hip_load takes. NULL with the reference's diagnostic
 * ("file:line: message") in tg_hip_error() for a model the reference
 * rejects, and for operations the batch backend does not run (autodiff,
 * training, sparse and memory operations, topk, suffix matching). Needs no
 * GPU. Free with tg_hip_str_free. */
char *tg_hip_surface_to_tgir(const char *path);

void tg_hip_free(tg_hip_prog *p);
const char *tg_hip_error(void);
int tg_hip_stats(const tg_hip_prog *p, tg_hip_stats_t *st);
int tg_hip_reset_stats(tg_hip_prog *p);

/* RTN quantization of a rank-2 f32 param on the host, as `tgc quantize
 * --method rtn` does it (src/quant.c:176-200, :258-316): per output channel
 * (axis 0: rows, W[C][K]; axis 1: columns, W[K][C]) the best of ten clipped
 * scales, codes in [-7, 7] or [-127, 127] one int8 per element in w's layout,
 * one f32 scale per channel. Channels are spread over `threads` threads. No
 * device is used. 0 on success, -1 on bad arguments. */
int tg_hip_quantize_rtn(const float *w, int rows, int cols, int bits, int axis, signed char *codes, float *scales, int threads);

/* KV-cache greedy decoding for models in the layout of the reference's Qwen3
 * importer (examples/qwen3/import.py:46-130: params E, LM, Rot, lnf, ln1_l,
 * ln2_l, qn_l, kn_l, Wq_l_h, Wk_l_j, Wv_l_j, Wo_l_h, Wg_l, Wu_l, Wd_l, all
 * matmul weights quantized on axis 1), plus RoPE tables `rope_cos` and
 * `rope_sin` with a row per position. No counterpart in the reference, which
 * runs such a model at one fixed length and has no cache: for callers that
 * generate text. Each generated token's logits equal the fixed-length forward's
 * at that position, bit for bit (finite activations). The decoder packs its
 * own copy of the weights and sizes its cache for max_seqs x max_len
 * positions; the program p must outlive it. */
typedef struct tg_hip_dec tg_hip_dec;
tg_hip_dec *tg_hip_dec_create(const tg_hip_prog *p, int max_seqs, int max_prompt, int max_len);
/* Prompts d_prompt [seqs][prompt_len] (f32 token ids, device memory): prefill,
 * then `steps` greedy tokens per sequence into d_tokens [seqs][steps] (int32,
 * device; may be NULL), the logits of each step into d_logits
 * [steps][seqs][vocab] (device; may be NULL). Asynchronous on the program's
 * stream (tg_hip_sync waits). 0 on success. */
int tg_hip_dec_generate(tg_hip_dec *d, const float *d_prompt, int seqs, int prompt_len, int steps, int *d_tokens, float *d_logits);
int tg_hip_dec_info(const tg_hip_dec *d, int *layers, int *vocab);
void tg_hip_dec_free(tg_hip_dec *d);

/* Device memory helpers for callers without their own allocator. */
void *tg_hip_dev_alloc(size_t bytes);
int tg_hip_dev_free(void *d);
/* Pinned (page-locked) host memory for rows, outputs and steps: tg_hip_batch
 * and tg_hip_batch_fixed move buffers that lie inside such an allocation over
 * PCIe directly, without their host-side staging copy, and `tgc-hip batch`
 * reads binary rows straight into it. No counterpart in the reference (its
 * rows live in ordinary memory, src/io.c:load_samples): for callers that
 * stream rows through the device. NULL on failure; tg_hip_host_free takes
 * only pointers from tg_hip_host_alloc (-1 otherwise). */
void *tg_hip_host_alloc(size_t bytes);
int tg_hip_host_free(void *h);
int tg_hip_h2d(void *d, const void *h, size_t bytes);
int tg_hip_d2h(void *h, const void *d, size_t bytes);
/* A read of `bytes` of device memory at d (16-byte aligned) that writes
 * nothing, asynchronous on `stream` (NULL: the null stream), in `blocks`
 * workgroups of 256 threads: the floor a bandwidth-bound kernel of that size
 * is measured against (the benchmark's matvec sweep). No counterpart in the
 * reference. 0 on success. */
int tg_hip_read_pass(const void *d, size_t bytes, int blocks, void *stream);

#ifdef __cplusplus
}
#endif
#endif
