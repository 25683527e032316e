// Host check of tg_log1p_unit (technograd_amd/csrc/tg_devmath.h): every
// STRIDE-th f32 in [0, 1] against the f32 rounding of the C library's f64
// log1p (correctly rounded away from rounding boundaries) and against the
// reference's f32 log1pf. Prints: values, differences from the correctly
// rounded value, differences from log1pf, largest of those in ulp.
#include "tg_devmath.h"

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>

int main(int argc, char **argv)
{
	const uint32_t stride = argc > 1 ? (uint32_t)strtoul(argv[1], nullptr, 10) : 1;
	const float one = 1.0f;
	uint32_t top;
	memcpy(&top, &one, 4);
	long n = 0, off_cr = 0, off_lib = 0, worst = 0;
	for (uint64_t b = 0; b <= top; b += stride) {
		const uint32_t w = (uint32_t)b;
		float y;
		memcpy(&y, &w, 4);
		const float a = tg_log1p_unit(y), cr = (float)log1p((double)y), lib = log1pf(y);
		n++;
		off_cr += a != cr;
		if (a != lib) {
			int32_t ia, il;
			memcpy(&ia, &a, 4);
			memcpy(&il, &lib, 4);
			off_lib++;
			if (labs((long)ia - il) > worst) worst = labs((long)ia - il);
		}
	}
	const float nan = tg_log1p_unit(NAN), zero = tg_log1p_unit(0.0f), l2 = tg_log1p_unit(1.0f);
	printf("%ld %ld %ld %ld %d %d %d\n", n, off_cr, off_lib, worst, std::isnan(nan) ? 1 : 0, zero == 0.0f && !std::signbit(zero),
	       l2 == (float)log(2.0));
	return 0;
}
