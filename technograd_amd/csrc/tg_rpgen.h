// Row programs compiled for one model: the emitter turns the flat row
// program of the row executor (tg_kern.h, rp_ins) into one HIP kernel in
// which every arena slot is a local variable (registers, not the [slot][lane]
// device arena), every param, constant, code and scale is a literal, and
// instructions of a think body whose operands do not change between
// iterations are hoisted in front of the loop. The kernel computes what the
// interpreter (kern_rowprog.hip) computes, element for element, through the
// same element functions (tg_rowdev.h).
#pragma once

#include "tg_kern.h"

#include <string>

// A row program and its pools on the host.
struct rp_source {
	const rp_ins *prog;
	int nins;
	const float *pool; // f32 words, or Q16.16 words stored in float slots
	long npool;
	const int *imap;
	const uint8_t *codes;
	const float *fscale;
	const int *qscale;
	int per, in_slot, nout, out_ref, nthink;
	long arena;
	bool fixed;
};

struct rp_emit_stats {
	long hoisted = 0;    // instructions moved in front of their think loop
	long terms = 0;      // multiply-add terms written out
	long slots = 0;      // arena slots that became variables
};

// The source of one translation unit holding
//   extern "C" __global__ void <kernel>(const T *in, T *out, int *steps, int rows)
// (T = int for Q16.16, float for f32; `in` is [rows][per], `out` [rows][nout],
// `steps` [rows][nthink] or null), self-contained: the element functions are
// part of the text. With `launcher`, it also holds a host entry point
//   extern "C" int <kernel>_batch(const void *d_in, int rows, void *d_out, int *d_steps, hipStream_t st)
// and compiles with hipcc as a standalone unit. Returns false, with the
// reason in `why`, for a program the compiled form does not take (scans,
// gathers, more slots or terms than registers and compile time allow).
bool rp_emit(const rp_source &s, const char *kernel, bool launcher, std::string &src, std::string &why, rp_emit_stats *st);
