// Runs a row-program unit emitted by tg_hip_emit_unit as host code: the
// kernel body is plain C++ over the element functions of tg_rowdev.h, so with
// the few launch built-ins below it compiles with g++ and runs row by row on
// the CPU (a check of the emitter that needs no GPU).
//   build: g++ -DTG_UNIT_FILE='"unit.hip"' -DTG_KERNEL=name -DTG_T=int|float
//   run:   unit_host IN.bin OUT.bin STEPS.bin ROWS PER NOUT NTHINK
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#define __global__
#define __device__
#define __launch_bounds__(n)
struct tg_dim {
	unsigned x, y, z;
};
static tg_dim blockIdx, threadIdx;
static inline float __int_as_float(int i)
{
	float f;
	memcpy(&f, &i, 4);
	return f;
}
#define TG_UNIT_KERNEL_ONLY
#include TG_UNIT_FILE

static bool io(const char *path, void *p, size_t n, bool write)
{
	FILE *f = fopen(path, write ? "wb" : "rb");
	if (!f) return false;
	size_t k = write ? fwrite(p, 1, n, f) : fread(p, 1, n, f);
	fclose(f);
	return k == n;
}

int main(int argc, char **argv)
{
	if (argc != 8) return 2;
	const long rows = atol(argv[4]), per = atol(argv[5]), nout = atol(argv[6]), nthink = atol(argv[7]);
	std::vector<TG_T> in((size_t)rows * per), out((size_t)rows * nout);
	std::vector<int> steps((size_t)rows * nthink);
	if (!io(argv[1], in.data(), in.size() * sizeof(TG_T), false)) return 3;
	for (long r = 0; r < rows; r++) {
		blockIdx.x = (unsigned)(r / 256);
		threadIdx.x = (unsigned)(r % 256);
		TG_KERNEL(in.data(), out.data(), steps.data(), (int)rows);
	}
	if (!io(argv[2], out.data(), out.size() * sizeof(TG_T), true)) return 4;
	if (!io(argv[3], steps.data(), steps.size() * sizeof(int), true)) return 5;
	return 0;
}
