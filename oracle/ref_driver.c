/* TEST INFRASTRUCTURE ONLY — driver for the reference build in oracle/_ref.
 *
 * Linked by oracle/Makefile against the reference's own sources, compiled
 * where they lie under /root/reference (src/util.c sexp.c ops.c parse.c
 * lower.c ir.c plan.c vm.c io.c trace.c par.c autodiff.c optim.c quant.c
 * serve.c). The reference's src/main.c is not linked: it also pulls in the C
 * and assembly code generators and the fixer, whose headers are generated at
 * build time (Makefile:15-27), so this file supplies the entry point instead.
 * Every computation is the reference's: load_module/plan/vm_run_into/par_for
 * for `batch` (restating the block loop of src/main.c:400-444 around them),
 * quantize_main for `quantize`, ir_write for `ir`, and runtime/tg_rtq.h's
 * kernels (ref_fixed.c) for `fixed`.
 *
 *   tgc_ref ir MODEL                                  canonical TGIR on stdout
 *   tgc_ref quantize MODEL [-o OUT] [--bits B] ...    the reference quantizer
 *   tgc_ref batch MODEL ROWS.bin -o OUT.bin [-j N] [--steps S.bin] [--fixed]
 *       ROWS: raw f32 (or raw int32 Q16.16 with --fixed); OUT likewise;
 *       S: raw int32 steps per row and think loop. Prints the compute time
 *       (ms), the wall time from before the input load to after the last
 *       write (the reference's `batch` trace, src/main.c:413-443) and the
 *       threads on stderr as `ref-batch rows R threads T ms M wall_ms W`.
 *   tgc_ref c MODEL -o UNIT.c [--fixed] [--harness MAIN.c]
 *       the reference's C generator (src/cgen.c, cgen_mode) on the loaded and
 *       planned module, as `tgc c` runs it (src/main.c:446-470). --harness
 *       also writes a driver of this file's own that includes UNIT.c and runs
 *       tg_<model>_run over raw rows: `main ROWS OUT STEPS` reads each row's
 *       inputs (raw words, in input order), writes the raw output words and
 *       the int32 tg_<model>_steps values (one per think loop, at least one). */
#include "tg.h"

#include <stdlib.h>
#include <string.h>
#include <time.h>

void ref_fixed_prepare(const Module *m);
void ref_fixed_run(const Module *m, const int *in, int *out, int *steps, int *arena);

typedef struct {
	const Module *m;
	const float *all;
	const int *alli;
	int per, n, nt, fixed;
	float *out;
	int *outi;
	int *steps;
	float *arenas;
	int afl;
	const float **inptrs;
} Job;

static void rows_fn(void *ctx, int lo, int hi, int tid)
{
	Job *j = ctx;
	const Module *m = j->m;
	float *arena = j->arenas + (size_t)tid * (size_t)j->afl;
	for (int r = lo; r < hi; r++) {
		if (j->fixed) {
			ref_fixed_run(m, j->alli + (size_t)r * j->per, j->outi + (size_t)r * j->n, j->steps + (size_t)r * j->nt, (int *)arena);
			continue;
		}
		const float **in = j->inptrs + (size_t)tid * (size_t)(m->ninputs ? m->ninputs : 1);
		const float *row = j->all + (size_t)r * (size_t)j->per;
		for (int i = 0, o = 0; i < m->ninputs; i++) {
			in[i] = row + o;
			o += shape_numel(&m->val[m->inputs[i]].sh);
		}
		vm_run_into(m, in, j->out + (size_t)r * (size_t)j->n, j->steps + (size_t)r * (size_t)j->nt, arena, NULL);
	}
}

static double now_ms(void)
{
	struct timespec t;
	clock_gettime(CLOCK_MONOTONIC, &t);
	return t.tv_sec * 1e3 + t.tv_nsec / 1e6;
}

static int batch(int argc, char **argv)
{
	const char *model = NULL, *data = NULL, *opath = NULL, *spath = NULL;
	int threads = 1, fixed = 0;
	for (int i = 2; i < argc; i++) {
		if (!strcmp(argv[i], "-o") && i + 1 < argc) opath = argv[++i];
		else if (!strcmp(argv[i], "--steps") && i + 1 < argc) spath = argv[++i];
		else if (!strcmp(argv[i], "-j") && i + 1 < argc) {
			i++;
			threads = strcmp(argv[i], "auto") == 0 ? 0 : atoi(argv[i]);
		} else if (!strcmp(argv[i], "--fixed")) fixed = 1;
		else if (!model) model = argv[i];
		else if (!data) data = argv[i];
		else die(NULL, 0, "unexpected argument '%s'", argv[i]);
	}
	if (!model || !data || !opath) die(NULL, 0, "usage: tgc_ref batch MODEL ROWS.bin -o OUT.bin [-j N] [--steps S.bin] [--fixed]");
	par_init(threads);
	Module *m = load_module(model);
	plan(m);
	if (m->nupd) die(NULL, 0, "model updates state: not a batch workload here");
	if (fixed) ref_fixed_prepare(m);
	int per = 0;
	for (int i = 0; i < m->ninputs; i++) per += shape_numel(&m->val[m->inputs[i]].sh);
	int n = shape_numel(&m->val[m->output].sh), nt = m->nthink ? m->nthink : 1;
	int cnt;
	double w0 = now_ms(); /* wall time as the reference's batch trace takes it: input load to last write (src/main.c:413-443) */
	float *all = io_load(data, &cnt); /* raw little-endian 32-bit words */
	if (cnt % per) die(NULL, 0, "'%s': %d values is not a multiple of the %d per sample", data, cnt, per);
	int rows = cnt / per, th = par_threads(), afl = m->arena ? m->arena : 1;
	Job j = { m, all, (const int *)all, per, n, nt, fixed, malloc((size_t)(rows ? rows : 1) * n * 4), NULL,
		  calloc((size_t)(rows ? rows : 1) * nt, sizeof(int)), malloc((size_t)th * afl * 4), afl,
		  malloc((size_t)th * (size_t)(m->ninputs ? m->ninputs : 1) * sizeof(float *)) };
	j.outi = (int *)j.out;
	double t0 = now_ms();
	int block = 1024 * th;
	for (int b0 = 0; b0 < rows; b0 += block) { /* blocks of 1024 x threads rows, as src/main.c:423-436 */
		int c = rows - b0 < block ? rows - b0 : block;
		int grain = c / (16 * th);
		Job jb = j;
		jb.all = all + (size_t)b0 * per;
		jb.alli = (const int *)all + (size_t)b0 * per;
		jb.out = j.out + (size_t)b0 * n;
		jb.outi = j.outi + (size_t)b0 * n;
		jb.steps = j.steps + (size_t)b0 * nt;
		par_for(c, grain > 0 ? grain : 1, rows_fn, &jb);
	}
	double ms = now_ms() - t0;
	FILE *f = fopen(opath, "wb");
	if (!f) die(NULL, 0, "cannot write '%s'", opath);
	fwrite(j.out, 4, (size_t)rows * n, f);
	if (fclose(f)) die(NULL, 0, "write failed '%s'", opath);
	if (spath) {
		f = fopen(spath, "wb");
		if (!f) die(NULL, 0, "cannot write '%s'", spath);
		fwrite(j.steps, sizeof(int), (size_t)rows * nt, f);
		if (fclose(f)) die(NULL, 0, "write failed '%s'", spath);
	}
	fprintf(stderr, "ref-batch rows %d threads %d ms %.3f wall_ms %.3f\n", rows, th, ms, now_ms() - w0);
	return 0;
}

/* The raw-row driver for a unit: every input row in, every output and steps
 * word out, with no decimal conversion in between. */
static void write_harness(const Module *m, const char *unit, FILE *f, int fixed)
{
	const char *ty = fixed ? "tg_t" : "float", *nm = m->name;
	int outn = shape_numel(&m->val[m->output].sh);
	fprintf(f, "/* raw-row driver for the generated unit %s (written by oracle/ref_driver.c) */\n", unit);
	fprintf(f, "#include \"%s\"\n#include <stdio.h>\n\n", unit);
	fputs("int main(int argc, char **argv)\n{\n", f);
	for (int i = 0; i < m->ninputs; i++) fprintf(f, "\tstatic %s in%d[%d];\n", ty, i, shape_numel(&m->val[m->inputs[i]].sh));
	fprintf(f, "\tstatic %s out[%d];\n", ty, outn);
	fputs("\tif (argc != 4) { fputs(\"usage: main ROWS OUT STEPS\\n\", stderr); return 2; }\n", f);
	fputs("\tFILE *fi = fopen(argv[1], \"rb\"), *fo = fopen(argv[2], \"wb\"), *fs = fopen(argv[3], \"wb\");\n", f);
	fputs("\tif (!fi || !fo || !fs) { fputs(\"cannot open files\\n\", stderr); return 2; }\n", f);
	fputs("\tfor (long r = 0;; r++) {\n", f);
	for (int i = 0; i < m->ninputs; i++) {
		int n = shape_numel(&m->val[m->inputs[i]].sh);
		fprintf(f, "\t\tif (fread(in%d, sizeof in%d[0], %d, fi) != %d) { if (%d == 0 && feof(fi)) break; fputs(\"short row\\n\", stderr); return 2; }\n",
			i, i, n, n, i);
	}
	if (m->ninputs == 0) fputs("\t\tif (r == 1) break;\n", f);
	fprintf(f, "\t\ttg_%s_run(", nm);
	for (int i = 0; i < m->ninputs; i++) fprintf(f, "in%d, ", i);
	fputs("out);\n", f);
	fprintf(f, "\t\tfwrite(out, sizeof out[0], %d, fo);\n", outn);
	fprintf(f, "\t\tfwrite(tg_%s_steps, sizeof(int), %d, fs);\n", nm, m->nthink ? m->nthink : 1);
	fputs("\t}\n\treturn fclose(fo) || fclose(fs) ? 1 : 0;\n}\n", f);
}

static int unit(int argc, char **argv)
{
	const char *model = NULL, *opath = NULL, *hpath = NULL;
	int fixed = 0;
	for (int i = 2; i < argc; i++) {
		if (!strcmp(argv[i], "-o") && i + 1 < argc) opath = argv[++i];
		else if (!strcmp(argv[i], "--harness") && i + 1 < argc) hpath = argv[++i];
		else if (!strcmp(argv[i], "--fixed")) fixed = 1;
		else if (!model) model = argv[i];
		else die(NULL, 0, "unexpected argument '%s'", argv[i]);
	}
	if (!model || !opath) die(NULL, 0, "usage: tgc_ref c MODEL -o UNIT.c [--fixed] [--harness MAIN.c]");
	Module *m = load_module(model);
	plan(m);
	FILE *f = fopen(opath, "w");
	if (!f) die(NULL, 0, "cannot write '%s'", opath);
	cgen_mode(m, f, fixed);
	if (fclose(f)) die(NULL, 0, "write failed '%s'", opath);
	if (hpath) {
		const char *base = strrchr(opath, '/');
		f = fopen(hpath, "w");
		if (!f) die(NULL, 0, "cannot write '%s'", hpath);
		write_harness(m, base ? base + 1 : opath, f, fixed);
		if (fclose(f)) die(NULL, 0, "write failed '%s'", hpath);
	}
	return 0;
}

int main(int argc, char **argv)
{
	if (argc < 3) {
		fputs("usage: tgc_ref ir|quantize|batch|c|serve|stream MODEL ...\n", stderr);
		return 2;
	}
	if (!strcmp(argv[1], "quantize")) {
		par_init(1);
		return quantize_main(argc, argv);
	}
	if (!strcmp(argv[1], "ir")) {
		Module *m = load_module(argv[2]);
		plan(m);
		ir_write(m, stdout);
		return 0;
	}
	if (!strcmp(argv[1], "batch")) return batch(argc, argv);
	if (!strcmp(argv[1], "c")) return unit(argc, argv);
	if (!strcmp(argv[1], "serve") || !strcmp(argv[1], "stream")) { /* src/main.c:361-369: the reference's connections */
		Module *m = load_module(argv[2]);
		plan(m);
		par_init(1);
		tg_signals();
		if (!strcmp(argv[1], "serve")) {
			if (argc != 5 || strcmp(argv[3], "--listen")) return 2;
			return serve_main(m, argv[4]);
		}
		const char *src = "-", *dst = NULL;
		for (int i = 3; i < argc; i++) {
			if (!strcmp(argv[i], "-o") && i + 1 < argc) dst = argv[++i];
			else src = argv[i];
		}
		return stream_main(m, src, dst);
	}
	fputs("unknown command\n", stderr);
	return 2;
}
