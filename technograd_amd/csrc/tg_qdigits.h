// Activation digits of the exact int8 matrix-core GEMM (kern_qgemm.hip), as
// device functions shared by the GEMM's digit kernels and the fused decode
// kernels, so every producer writes the same bytes.
//
// A row x of K inputs is written as q_k = rint(x_k 2^(23-E)), E the row's
// exponent (max |x| = f 2^E, f in [0.5, 1), raised by one when the top digit
// would leave int8), and each q as three balanced base-256 int8 digits. Rows
// with a non-finite entry or max |x| above 2^100 are "special": their digits
// are zero and the GEMM's epilogue runs the reference's sequential loop.
//
// Rows whose grid is too coarse. The grid step 2^(E-23) is set by the
// largest entry; when a few entries stand far above the others (outlier
// channels), the others lose precision on that grid, and if the outliers
// meet zero codes the product's own size no longer hides that loss. Every
// producer tallies, per row, the sum of |q| over the row's grid and the
// number n of inexact entries (x 2^(23-E) not an integer). A row is a
// candidate when some entry is inexact and sum |q| < (J(n) + A(n)) 2^23,
// with J(n) = clamp(n / 16, 1, 64) (how many of the largest entries may be
// outliers) and A(n) = ceil(3 isqrt(n) / 4) (the grid's random rounding
// error over n inexact entries, with a margin). Candidates take the
// reference's loop until they are resolved (tgq_decide, a wave per row):
// over a histogram of the row's binades below E, the smallest peel level L
// (entries |x| >= 2^(E-L) become exact outlier terms, at most J of them) at
// which the rest, less its own J largest entries, still holds A(n) grid
// steps of its own. Level 0 keeps the row on its grid, a level L > 0 splits
// it (the outliers as exact terms, the rest on a grid of its own), and no
// level leaves it with the reference's loop. Every quantity is an integer
// count or sum, so the decision does not depend on the order of any sum, nor
// on which kernel or batch size makes it: a row gets the same bits in every
// batch.
//
// Layout (the MFMA fragment order of v_mfma_i32_32x32x32_i8):
//   digits [row / 32][k / 32][digit 0..2][lane 0..63][16 bytes],
//   lane = row % 32 + 32 ((k % 32) / 16).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef int tgq_v4i __attribute__((ext_vector_type(4)));

// balanced base-256 digits of |q| < 2^23: q = d0 + 256 d1 + 65536 d2, d_l in [-128, 127]
__device__ inline void tgq_split3(int q, int &d0, int &d1, int &d2)
{
	d0 = (int)(int8_t)(q & 255);
	const int q1 = (q - d0) >> 8;
	d1 = (int)(int8_t)(q1 & 255);
	d2 = (q1 - d1) >> 8;
}

// a row is special when an entry is not finite (bad) or max |x| exceeds 2^100
__device__ inline int tgq_special(int bad, float amax) { return bad || amax > 0x1p100f; }

// A row's class in a digit area's special flags. Consumers take the
// reference's loop for any odd flag, so a candidate that no resolve has seen
// still gets an exact result.
enum { TGQ_GRID = 0, TGQ_REF = 1, TGQ_SPLIT = 2, TGQ_CAND = 3 };

// The candidate tally: sum |q| in bits 0..43 (|q| <= 2^23, at most 2^19
// inputs) plus the count of inexact entries from bit 44.
constexpr int TGQ_TALLY_SHIFT = 44;
constexpr int TGQ_MAX_OUT = 64;  // outliers of a split row, at most
constexpr int TGQ_MASS_SHIFT = 44; // the histogram's mass unit: 2^(E-44)

__device__ inline int tgq_isqrt(int n)
{
	int r = (int)sqrtf((float)n); // then corrected: exact whatever the rounding of sqrtf
	while (r > 0 && r * r > n) r--;
	while ((r + 1) * (r + 1) <= n) r++;
	return r;
}
__device__ inline int tgq_jcap(int n) { return n < 32 ? 1 : n >= 16 * TGQ_MAX_OUT ? TGQ_MAX_OUT : n >> 4; }
__device__ inline int tgq_acoef(int n) { return (3 * tgq_isqrt(n) + 3) >> 2; }
// outlier slots per row of a digit area of Kp inputs (J(n) <= K / 16 <= this)
__host__ __device__ inline int tgq_nout(int Kp) { return Kp >= 16 * TGQ_MAX_OUT ? TGQ_MAX_OUT : Kp >> 4 < 1 ? 1 : Kp >> 4; }

// the tally of 16 inputs on the grid of exponent E
__device__ inline long long tgq_tally16(const float *v, int E)
{
	int aq = 0, nx = 0;
	for (int i = 0; i < 16; i++) {
		const float sv = ldexpf(v[i], 23 - E), rq = rintf(sv);
		aq += abs((int)rq);
		nx += rq != sv;
	}
	return (long long)aq + ((long long)nx << TGQ_TALLY_SHIFT);
}
__device__ inline int tgq_candidate(long long tally)
{
	const int n = (int)(tally >> TGQ_TALLY_SHIFT);
	if (n == 0) return 0; // every entry on the grid: the product is exact
	const long long mass = tally & ((1ll << TGQ_TALLY_SHIFT) - 1);
	return mass < ((long long)(tgq_jcap(n) + tgq_acoef(n)) << 23);
}

// the row exponent E from max |x| (0 for special or all-zero rows)
__device__ inline int tgq_exponent(float amax, int special)
{
	int E = 0;
	if (!special && amax > 0.0f) {
		frexpf(amax, &E); // amax = f 2^E, f in [0.5, 1)
		if (rintf(ldexpf(amax, 23 - E)) > 8355328.0f) E += 1; // keep the top digit within int8
	}
	return E;
}

// row m's first fragment byte in a digit area of Kp inputs per row
__device__ inline int8_t *tgq_row_base(int8_t *dig, int m, int Kp) { return dig + (long)(m >> 5) * (Kp / 32) * 3072 + (m & 31) * 16; }

// Row scan: the running max of |x| over a lane's inputs, kept as the bit
// pattern of |x| (unsigned order is the order of magnitudes, and every NaN
// pattern lies above +inf's 0x7f800000): two inputs per max3, no compare.
__device__ inline void tgq_scan16(const float *v, unsigned &mb)
{
	for (int i = 0; i < 16; i += 2) {
		const unsigned a = __float_as_uint(v[i]) & 0x7fffffffu, b = __float_as_uint(v[i + 1]) & 0x7fffffffu;
		mb = max(mb, max(a, b));
	}
}

// four inputs' u = q + 0x808080 -> their digit bytes in the three plane words
// (byte i of plane l's word: d_l of input i; the layout tgq_put16 writes)
__device__ inline void tgq_pack4(const unsigned *u, unsigned &w0, unsigned &w1, unsigned &w2)
{
	const unsigned t01 = __builtin_amdgcn_perm(u[1], u[0], 0x05010400u); // u0.b0 u1.b0 u0.b1 u1.b1
	const unsigned t23 = __builtin_amdgcn_perm(u[3], u[2], 0x05010400u); // u2.b0 u3.b0 u2.b1 u3.b1
	const unsigned s01 = __builtin_amdgcn_perm(u[1], u[0], 0x0c0c0602u); // u0.b2 u1.b2 0 0
	const unsigned s23 = __builtin_amdgcn_perm(u[3], u[2], 0x06020c0cu); // 0 0 u2.b2 u3.b2
	w0 = __builtin_amdgcn_perm(t23, t01, 0x05040100u) ^ 0x80808080u;
	w1 = __builtin_amdgcn_perm(t23, t01, 0x07060302u) ^ 0x80808080u;
	w2 = (s01 | s23) ^ 0x80808080u;
}

// a lane's max |x| and NaN flag from its scan (a NaN lane's max is not used:
// the flag makes the row special). An infinite input is not flagged here: it
// makes max |x| infinite, which tgq_special treats as special all the same.
__device__ inline void tgq_scan_end(unsigned mb, float &mx, int &nan)
{
	nan = mb > 0x7f800000u;
	mx = nan ? 0.0f : __uint_as_float(mb);
}

// the digit words of 16 consecutive inputs: w_l[g] holds plane l's digits of
// inputs 4 g .. 4 g + 3 (byte i: input 4 g + i); returns the sum of q and
// adds the inputs' candidate tally (tgq_tally16) to `tally`.
// With u = q + 0x808080 (|q| <= 8355328, so 0 <= u < 2^24), byte l of u is
// d_l + 128: the balanced digits are u's bytes with the top bit flipped. The
// bytes of four inputs are gathered into each plane's 32-bit word with byte
// permutes (v_perm_b32 selects bytes of a register pair: 0-3 the second
// operand's, 4-7 the first's, 12 a zero byte).
__device__ inline long long tgq_digits16(const float *v, int E, unsigned (&w0)[4], unsigned (&w1)[4], unsigned (&w2)[4], long long &tally)
{
	int qs = 0, aq = 0, nx = 0; // |sum of 16 q| < 2^27
	for (int g = 0; g < 4; g++) {
		unsigned u[4];
		for (int i = 0; i < 4; i++) {
			const float sv = ldexpf(v[4 * g + i], 23 - E), rq = rintf(sv);
			const int q = (int)rq; // exact: |q| < 2^23
			qs += q;
			aq += abs(q);
			nx += rq != sv;
			u[i] = (unsigned)(q + 0x808080);
		}
		tgq_pack4(u, w0[g], w1[g], w2[g]);
	}
	tally += (long long)aq + ((long long)nx << TGQ_TALLY_SHIFT);
	return qs;
}

// digits of 16 consecutive inputs (inputs k0 .. k0 + 15 of the row at blk)
// into their three 16-byte chunks of the fragment layout; zero digits when
// `zero`; returns the sum of q and adds the inputs' candidate tally to
// `tally` (nothing for a `zero` group).
__device__ inline long long tgq_put16(int8_t *blk, int k0, const float *v, int E, bool zero, long long &tally)
{
	int8_t *p = blk + (k0 >> 5) * 3072 + ((k0 >> 4) & 1) * 512;
	if (__builtin_expect(zero, 0)) {
		*(tgq_v4i *)p = tgq_v4i{0, 0, 0, 0};
		*(tgq_v4i *)(p + 1024) = tgq_v4i{0, 0, 0, 0};
		*(tgq_v4i *)(p + 2048) = tgq_v4i{0, 0, 0, 0};
		return 0;
	}
	unsigned w0[4], w1[4], w2[4];
	const long long qs = tgq_digits16(v, E, w0, w1, w2, tally);
	*(tgq_v4i *)p = tgq_v4i{(int)w0[0], (int)w0[1], (int)w0[2], (int)w0[3]};
	*(tgq_v4i *)(p + 1024) = tgq_v4i{(int)w1[0], (int)w1[1], (int)w1[2], (int)w1[3]};
	*(tgq_v4i *)(p + 2048) = tgq_v4i{(int)w2[0], (int)w2[1], (int)w2[2], (int)w2[3]};
	return qs;
}

// ---- resolving a candidate row (a whole wave) ----

__device__ inline int tgq_wave_sum(int v)
{
	for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
	return v;
}

// orders this wave's LDS writes and atomics before its later LDS reads of
// other lanes' words: every LDS operation issued so far has completed
__device__ inline void tgq_wave_sync()
{
	asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
	__builtin_amdgcn_wave_barrier();
}

// A row's histogram over the binades below its grid's exponent E: bin d holds
// the nonzero entries with 2^(E-d-1) <= |x| < 2^(E-d) (d = E - frexp
// exponent, clamped to 63), their count and the sum of floor(|x| 2^(44-E))
// (each term an exact integer below 2^44). P and PM are the bins' prefix
// sums: P[L] entries, PM[L] mass in bins below L.
struct TgqHist {
	unsigned cnt[64];
	unsigned bmax[64]; // the bin's largest |x| (as bits: non-negative floats order as their bits)
	unsigned long long mass[64];
	unsigned P[65];
	unsigned long long PM[65];
};

__device__ inline int tgq_bin(float ax, int E) // ax > 0, finite, below 2^E (so E - e >= 0; clamped all the same)
{
	int e;
	frexpf(ax, &e);
	const int d = E - e;
	return d < 0 ? 0 : d > 63 ? 63 : d;
}

// whether x is an outlier at peel level L: nonzero in a bin below L (|x| >= 2^(E-L))
__device__ inline bool tgq_outlier(float x, int E, int L) { return x != 0.0f && tgq_bin(fabsf(x), E) < L; }

// adds 16 inputs to the histogram (LDS atomics: integer sums, any order);
// returns how many of them are inexact on the grid of E
__device__ inline int tgq_hist16(TgqHist *h, const float *v, int E)
{
	int nx = 0;
	for (int i = 0; i < 16; i++) {
		const float ax = fabsf(v[i]);
		if (ax == 0.0f) continue;
		const float sv = ldexpf(v[i], 23 - E);
		nx += rintf(sv) != sv;
		const int d = tgq_bin(ax, E);
		atomicAdd(&h->cnt[d], 1u);
		atomicMax(&h->bmax[d], __float_as_uint(ax));
		atomicAdd(&h->mass[d], (unsigned long long)ldexpf(ax, TGQ_MASS_SHIFT - E)); // truncation: the floor
	}
	return nx;
}

// The peel level of a candidate with n inexact entries from its histogram
// (lane L tests level L): the smallest L with at most J = J(n) entries in
// bins below L such that the rest, less its J largest entries, still holds
// A(n) units of its top bin r's 2^(E-r). The J largest are taken bin by bin
// from r; a bin taken in part counts each taken entry at the bin's upper end.
// A rest with nothing in it is enough; a top bin past 44 (a mass unit below
// 1) is not. Returns -1 when no level is enough.
__device__ inline int tgq_decide(TgqHist *h, int n, int lane)
{
	const int J = tgq_jcap(n);
	const long long A = tgq_acoef(n);
	const unsigned c = h->cnt[lane];
	const unsigned long long ms = h->mass[lane];
	unsigned pc = c; // inclusive prefix sums over the bins
	unsigned long long pm = ms;
	for (int o = 1; o < 64; o <<= 1) {
		const unsigned t = __shfl_up(pc, o);
		const unsigned long long tm = __shfl_up(pm, o);
		if (lane >= o) pc += t, pm += tm;
	}
	h->P[lane + 1] = pc;
	h->PM[lane + 1] = pm;
	if (lane == 0) h->P[0] = 0, h->PM[0] = 0;
	tgq_wave_sync();
	const unsigned PL = pc - c;                               // entries in bins below L
	const unsigned long long SL = __shfl(pm, 63) - (pm - ms); // mass in bins L and up
	const unsigned long long rest = __ballot(c != 0) >> lane;
	bool ok = false;
	if (PL <= (unsigned)J) {
		if (rest == 0) {
			ok = true;
		} else {
			const int r = lane + __builtin_ctzll(rest);
			if (r <= TGQ_MASS_SHIFT) {
				const unsigned target = h->P[r] + (unsigned)J;
				long long top;
				if (h->P[64] <= target) {
					top = (long long)SL; // the rest is J entries or fewer
				} else {
					int lo = r, hi = 63; // the bin where the J largest end: P[lo + 1] >= target
					while (lo < hi) {
						const int mid = (lo + hi) >> 1;
						if (h->P[mid + 1] >= target) hi = mid;
						else lo = mid + 1;
					}
					top = h->P[lo + 1] == target ? (long long)(h->PM[lo + 1] - h->PM[r])
								    : (long long)(h->PM[lo] - h->PM[r]) +
									      (lo <= TGQ_MASS_SHIFT ? (long long)(target - h->P[lo]) << (TGQ_MASS_SHIFT - lo) : 0ll);
				}
				ok = (long long)SL - top >= A << (TGQ_MASS_SHIFT - r);
			}
		}
	}
	const unsigned long long okm = __ballot(ok);
	return okm ? __builtin_ctzll(okm) : -1;
}

// ---- the producers' coarse test ----
//
// Most candidates keep their grid when resolved. A producer settles most of
// those without a resolve by a coarse test on integers it has at hand: the
// row's q = rint(x 2^(23-E)) sorted into three groups, |q| >= 2^22 (holding
// TgqHist's bin 0 and entries just below it), 2^21 <= |q| < 2^22 (the rest
// of bin 1 and entries just below it) and the other nonzero entries (every
// entry of bins 2 and up), with the groups' counts and sums of |q|, plus the
// tally's sum of |q| and inexact count. tgq_coarse_grid runs tgq_decide's
// level-0 test on the groups with bounds: a group taken whole counts each
// entry at (|q| + 1/2) 2^21 (at least its mass floor(|x| 2^(44-E)); 2^20 for
// a nonzero entry with q = 0), a group taken in part counts each taken entry
// at the group's upper end (2^44, 2^43, 2^42: no entry of the group has more
// mass), the row's mass counts as sum (|q| - 1/2) 2^21 over nonzero entries
// (at most the true mass), and the rest's top bin is the first nonempty
// group's index (no entry's group index exceeds its bin). So the coarse top
// mass is at least tgq_decide's, the coarse rest mass at most its, and the
// coarse top bin at most its: a row that passes here passes tgq_decide at
// level 0, where the resolve leaves a row as it is, and a row's class is the
// same whether or not its producer runs this test first.
struct TgqCoarse {
	unsigned long long cnt;    // |q| >= 2^22: bits 0..20; 2^21 <= |q| < 2^22: bits 21..41; nonzero x: from bit 42
	unsigned long long s0, s1; // sums of |q| of the first two groups
};

__device__ inline void tgq_coarse_add(TgqCoarse &c, const TgqCoarse &o) { c.cnt += o.cnt, c.s0 += o.s0, c.s1 += o.s1; }

// adds 16 inputs of a row with grid exponent E (finite, below 2^E)
__device__ inline void tgq_coarse16(TgqCoarse &c, const float *v, int E)
{
	unsigned n0 = 0, n1 = 0, nz = 0, a0 = 0, a1 = 0; // |q| < 2^23: 16 of them below 2^27
	for (int i = 0; i < 16; i++) {
		const unsigned aq = (unsigned)abs((int)rintf(ldexpf(v[i], 23 - E)));
		const bool g0 = aq >= (1u << 22), g1 = !g0 && aq >= (1u << 21);
		n0 += g0, n1 += g1, nz += v[i] != 0.0f;
		a0 += g0 ? aq : 0u, a1 += g1 ? aq : 0u;
	}
	c.cnt += (unsigned long long)n0 + ((unsigned long long)n1 << 21) + ((unsigned long long)nz << 42);
	c.s0 += a0, c.s1 += a1;
}

__device__ inline TgqCoarse tgq_coarse_wave_sum(TgqCoarse c)
{
	for (int o = 32; o > 0; o >>= 1) c.cnt += __shfl_xor(c.cnt, o), c.s0 += __shfl_xor(c.s0, o), c.s1 += __shfl_xor(c.s1, o);
	return c;
}

// whether a candidate row with the tally `tally` keeps its grid by the coarse test alone
__device__ inline bool tgq_coarse_grid(const TgqCoarse &c, long long tally)
{
	const int n = (int)(tally >> TGQ_TALLY_SHIFT);
	const long long aq = tally & ((1ll << TGQ_TALLY_SHIFT) - 1); // sum of |q| over the row
	const unsigned long long lo21 = (1ull << 21) - 1;
	const long long c0 = (long long)(c.cnt & lo21), c1 = (long long)((c.cnt >> 21) & lo21), nz = (long long)(c.cnt >> 42);
	const long long cnt[3] = { c0, c1, nz - c0 - c1 };
	const long long sq[3] = { (long long)c.s0, (long long)c.s1, aq - (long long)c.s0 - (long long)c.s1 };
	const int r = cnt[0] ? 0 : cnt[1] ? 1 : 2;
	if (!cnt[r]) return false; // an all-zero row is no candidate
	long long left = tgq_jcap(n), top = 0;
	for (int d = r; d < 3 && left > 0; d++) {
		const long long take = cnt[d] < left ? cnt[d] : left;
		top += take == cnt[d] ? (sq[d] << 21) + (cnt[d] << 20) : take << (TGQ_MASS_SHIFT - d);
		left -= take;
	}
	const long long mass_lo = (aq << 21) - (nz << 20);
	return mass_lo - top >= (long long)tgq_acoef(n) << (TGQ_MASS_SHIFT - r);
}

// Resolves a candidate row of grid exponent E (a whole wave; h in LDS, this
// wave's own): ld(g, v) loads the row's 16-input group g of ng (zeros past
// the row). Returns the peel level: 0 the grid, L > 0 a split at level L
// (tgq_outlier), -1 the reference's loop.
template <class Ld>
__device__ inline int tgq_resolve(TgqHist *h, Ld ld, int ng, int E, int lane)
{
	h->cnt[lane] = 0;
	h->bmax[lane] = 0;
	h->mass[lane] = 0;
	tgq_wave_sync();
	int nx = 0;
	for (int g = lane; g < ng; g += 64) {
		float v[16];
		ld(g, v);
		nx += tgq_hist16(h, v, E);
	}
	tgq_wave_sync();
	return tgq_decide(h, tgq_wave_sum(nx), lane);
}

// Resolves candidate row m of a digit area in place (a whole wave; h this
// wave's own, in LDS): ld(g, v) loads the row's 16-input group g (zeros past
// K), E0 is the row's grid exponent, blk its first fragment byte (tgq_row_base).
// The row keeps its digits (TGQ_GRID), takes the reference's loop (TGQ_REF),
// or is split (TGQ_SPLIT): its rest's digits, exponent and sum of q are
// rewritten and its outliers (input index and value, increasing index, -1
// after the last) go to ok / ox [nout]. The rest's exponent comes from the
// largest |x| of its top bin, so the row is read once, or twice when split.
template <class Ld>
__device__ inline void tgq_resolve_row(TgqHist *h, Ld ld, int K, int Kp, int E0, int8_t *blk, long long *qsum, int *e, int *special,
				       int *ok, float *ox, int nout, int lane)
{
	const int ng = Kp / 16;
	const int L = tgq_resolve(h, ld, ng, E0, lane);
	if (L <= 0) {
		if (lane == 0) *special = L < 0 ? TGQ_REF : TGQ_GRID;
		return;
	}
	const unsigned long long restb = __ballot(lane >= L && h->cnt[lane] != 0);
	const float rmax = restb ? __uint_as_float(h->bmax[__builtin_ctzll(restb)]) : 0.0f;
	const int E = tgq_exponent(rmax, 0);
	long long qs = 0, tl = 0;
	int nin = 0;
	for (int g0 = 0; g0 < ng; g0 += 64) {
		const int g = g0 + lane;
		float v[16];
		if (g < ng) ld(g, v);
		else
			for (int i = 0; i < 16; i++) v[i] = 0.0f;
		unsigned om = 0;
		for (int i = 0; i < 16; i++)
			if (tgq_outlier(v[i], E0, L)) om |= 1u << i;
		float r[16];
		for (int i = 0; i < 16; i++) r[i] = (om >> i) & 1 ? 0.0f : v[i];
		if (g < ng) qs += tgq_put16(blk, g * 16, r, E, g * 16 >= K, tl);
		// the outliers in input order: an exclusive scan of the lanes' counts
		const int cnt = __popc(om);
		int inc = cnt;
		for (int d = 1; d < 64; d <<= 1) {
			const int t = __shfl_up(inc, d);
			if (lane >= d) inc += t;
		}
		int at = nin + inc - cnt;
		for (int i = 0; i < 16; i++)
			if ((om >> i) & 1) {
				if (at < nout) ok[at] = g * 16 + i, ox[at] = v[i];
				at++;
			}
		nin += __shfl(inc, 63);
	}
	for (int o = 32; o > 0; o >>= 1) qs += __shfl_xor(qs, o);
	for (int j = nin + lane; j < nout; j += 64) ok[j] = -1;
	if (lane == 0) *e = E, *qsum = qs, *special = TGQ_SPLIT;
}
