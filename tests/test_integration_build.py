"""Reference-side bindings of the tg_hip C ABI compile against the
reference's own declarations (src/tg.h, runtime/tg_rt.h) with the
reference's compiler flags (-std=c11 -Wall -Wextra -Wpedantic, Makefile:2)
and include/tg_hip.h: the batch block loop (the model written to memory
with ir_write through open_memstream, which needs the POSIX feature macro
under -std=c11), the per-instruction offload (tg_hip_matmul_qa /
tg_hip_matmul_qb with tg_matmul_qa / qb's argument lists), the surface front
end and quantization.
The file only has to compile: it is not linked (no GPU, no reference
build). Skipped where the reference sources are absent."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"

BINDINGS = r"""
#define _POSIX_C_SOURCE 200809L /* open_memstream under -std=c11 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "tg.h"
#include "tg_hip.h"
#include "tg_rt.h"

/* tgc batch: the model of a stateless batch on the device, or NULL (CPU path) */
tg_hip_prog *bind_load(const Module *m, int block)
{
	tg_hip_prog *hp = NULL;
	if (!m->nupd && !getenv("TG_NO_HIP") && tg_hip_init(0) == 0) {
		char *txt = NULL;
		size_t len = 0;
		FILE *ms = open_memstream(&txt, &len);
		if (!ms) return NULL;
		ir_write(m, ms);
		fclose(ms);
		hp = tg_hip_load(txt, len, 0, block);
		free(txt);
		if (!hp) fprintf(stderr, "tgc: GPU backend: %s; using the CPU\n", tg_hip_error());
	}
	return hp;
}

/* tgc batch: one block of rows */
void bind_block(tg_hip_prog *hp, const float *all, int per, int b0, int cnt, float *out, int *steps)
{
	if (tg_hip_batch(hp, all + (size_t)b0 * (size_t)per, cnt, out, steps) != 0) die(NULL, 0, "GPU batch: %s", tg_hip_error());
}

/* per-instruction offload: the quantized matmul of src/vm.c:277-281, the function name swapped */
void bind_matmul(float *o, const float *a, const float *c, const signed char *qa, int qabits, const float *qas,
		 const signed char *qb, int qbbits, const float *qbs, int mm, int kk, int nn, int left)
{
	if (left) {
		if (tg_hip_matmul_qa(o, qa, qabits, qas, c, mm, kk, nn) != 0) tg_matmul_qa(o, qa, qabits, qas, c, mm, kk, nn);
	} else {
		if (tg_hip_matmul_qb(o, a, qb, qbbits, qbs, mm, kk, nn) != 0) tg_matmul_qb(o, a, qb, qbbits, qbs, mm, kk, nn);
	}
}

/* a surface model straight to the device */
tg_hip_prog *bind_surface(const char *path, int block)
{
	char *txt = tg_hip_surface_to_tgir(path);
	tg_hip_prog *hp = txt ? tg_hip_load(txt, strlen(txt), 0, block) : NULL;
	tg_hip_str_free(txt);
	return hp;
}

/* tgc quantize on the backend */
int bind_quantize(const Module *m, int bits, int gptq, const float *rows, long nrows, int min_size, FILE *out)
{
	char *txt = NULL;
	size_t len = 0;
	FILE *ms = open_memstream(&txt, &len);
	if (!ms) return -1;
	ir_write(m, ms);
	fclose(ms);
	static char log[1 << 16];
	long bytes[2];
	char *q = tg_hip_quantize_model(txt, len, bits, gptq, rows, nrows, min_size, 2048, bytes, log, sizeof log);
	free(txt);
	fputs(log, stderr);
	if (!q) return -1;
	fputs(q, out);
	tg_hip_str_free(q);
	fprintf(stderr, "quantize: params %ld -> %ld bytes\n", bytes[0], bytes[1]);
	return 0;
}
"""


@pytest.mark.skipif(not os.path.exists(os.path.join(REF, "src", "tg.h")), reason="reference sources absent")
@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc absent")
def test_bindings_compile_against_the_reference(tmp_path):
    src = tmp_path / "bind.c"
    src.write_text(BINDINGS)
    r = subprocess.run(["gcc", "-std=c11", "-Wall", "-Wextra", "-Wpedantic", "-Werror", "-fsyntax-only",
                        "-I" + os.path.join(REF, "src"), "-I" + os.path.join(REF, "runtime"),
                        "-I" + os.path.join(ROOT, "include"), str(src)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
