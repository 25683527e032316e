// The f32 elementwise operations of the layer executor (runtime/tg_rt.h:40-75
// and the binary kernels), shared by the elementwise kernels and the GEMM
// epilogues that apply an instruction chain to their outputs, so a value
// computed in either place is the same bits. Compiled with
// -ffp-contract=off: every multiply and add rounds separately, as the
// reference's C does.
#pragma once

#include "tg_devmath.h"
#include "tg_kern.h"
#include "tgm.h"

#include <math.h>

__device__ inline float tg_bop(int op, float x, float y)
{
	switch (op) {
	case TGK_ADD: return x + y;
	case TGK_SUB: return x - y;
	case TGK_MUL: return x * y;
	case TGK_DIV: return x / y;
	case TGK_MAX: return x > y ? x : y;
	default: return x < y ? x : y;
	}
}

__device__ inline float tg_uop(int op, float x)
{
	switch (op) {
	case TGM_NEG: return -x;
	case TGM_TANH: return tanhf(x);
	case TGM_RELU: return x > 0.0f ? x : 0.0f;
	case TGM_SIGMOID: return 1.0f / (1.0f + expf(-x));
	case TGM_EXP: return expf(x);
	case TGM_SQRT: return sqrtf(x);
	case TGM_GELU: return 0.5f * x * (1.0f + tanhf(0.7978845608f * (x + 0.044715f * x * x * x)));
	case TGM_SILU: return x / (1.0f + expf(-x));
	case TGM_SOFTPLUS: return (x > 0.0f ? x : 0.0f) + tg_log1p_unit(expf(-fabsf(x)));
	case TGM_LOG: return logf(x);
	case TGM_SIN: return sinf(x);
	case TGM_COS: return cosf(x);
	case TGM_FLOOR: return floorf(x);
	default: return x > 0.0f ? 1.0f : 0.0f; // step
	}
}
