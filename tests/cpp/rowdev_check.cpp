// Host build of the row programs' Q16.16 element functions
// (technograd_amd/csrc/tg_rowdev.h, the header both row executors use),
// exported for a ctypes comparison against the oracle.
#define __device__
#include "tg_rowdev.h"

extern "C" long rowdev_prim(int op, long a, long b)
{
	using namespace tgrd;
	switch (op) {
	case 0: return fmulq((int)a, (int)b);
	case 1: return fdivq((int)a, (int)b);
	case 2: return expq((int)a);
	case 3: return logq((int)a);
	case 4: return (long)isqrt64((unsigned long)a);
	case 5: return sinq((int)a);
	case 6: return tanhq((int)a);
	case 7: return sigmoidq((int)a);
	case 8: return a >= 0 && a <= 8 ? expc((int)a) : 0;
	case 9: return softq(a, b);
	case 10: return qscaleq(a, (int)b);
	case 11: return rmsq((unsigned long)a, (int)b);
	case 12: return expq_neg((int)a);
	case 13: return fdivq_unit((int)a, (int)b);
	case 14: return addq((int)a, (int)b);
	case 15: return subq((int)a, (int)b);
	case 16: return absq((int)a);
	}
	return 0;
}

extern "C" long rowdev_const(int which)
{
	using namespace tgrd;
	const long v[] = { LN2, PIQ, HPIQ, TPIQ, GELU_A, GELU_B, (long)EPS_Q32, EXP_HI, EXP_LO };
	return which >= 0 && which < 9 ? v[which] : 0;
}

extern "C" void rowdev_prim_n(int op, const long *a, long *out, long n)
{
	for (long i = 0; i < n; i++) out[i] = rowdev_prim(op, a[i], 0);
}
