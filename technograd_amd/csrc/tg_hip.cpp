// tg_hip: device programs for Technograd models on MI355X, behind a C ABI.
//
// A model (TGIR text) becomes one of two device programs:
//
//  * layer program: every instruction is one kernel over a block of batch
//    rows; values of the block live as [rows][numel] in one device arena
//    (the reference's per-row static arena, src/plan.c:154-224, widened to a
//    block of rows and allocated once); quantized matmuls run on the int8
//    matrix cores (kern_qgemm.hip), everything else on the exact kernels of
//    kern_layer.hip. Scans step through time on the host, each step a few
//    kernels over all rows.
//  * row program: one lane per batch row runs the whole model. Used for
//    think loops (per-row halting), for Q16.16, and on request. The program
//    is compiled for the model at load time (tg_rpgen.cpp, hipRTC): values in
//    registers, weights as literals, loop-invariant instructions hoisted out
//    of think loops. Programs the compiled form does not take (scans,
//    gathers, very large rows) run in the row-program interpreter
//    (kern_rowprog.hip), which computes the same values.
//
// The batch loop mirrors `tgc batch` (src/main.c:400-444): rows are processed
// in blocks (here: device passes of up to max_rows rows), outputs come back in
// input order, and steps per row are reported for every think loop.
#include "tg_hip.h"
#include "tg_front.h"
#include "tg_gptq.h"
#include "tg_kern.h"
#include "tg_rpgen.h"
#include "tgm.h"

#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <algorithm>
#include <cctype>
#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

namespace {

thread_local char g_err[1024];

void seterr(const char *fmt, ...)
{
	va_list ap;
	va_start(ap, fmt);
	vsnprintf(g_err, sizeof g_err, fmt, ap);
	va_end(ap);
}

bool hipok(hipError_t e, const char *what)
{
	if (e == hipSuccess) return true;
	seterr("%s: %s", what, hipGetErrorString(e));
	return false;
}

// Scratch of tg_hip_matmul_q_noalloc: packed weights, padded scales and the
// activation digits of one call, in device memory every GPU the library runs
// on holds from module load until the process ends. In host code `scratch`
// is only a stand-in for the symbol: its device address on each GPU comes
// from hipGetSymbolAddress (scratch_on), and only that address is used.
static __device__ __align__(256) uint8_t scratch[TG_HIP_NOALLOC_SCRATCH];

constexpr int MAX_DEVICES = 64;
void *g_scratch[MAX_DEVICES]; // scratch's address on each device, set once by scratch_on

// scratch's address on `device` (the current device), looked up once per device
void *scratch_on(int device)
{
	if (device < 0 || device >= MAX_DEVICES) {
		seterr("device %d: beyond the %d devices the scratch table covers", device, MAX_DEVICES);
		return nullptr;
	}
	void *p = __atomic_load_n(&g_scratch[device], __ATOMIC_ACQUIRE);
	if (p) return p;
	if (!hipok(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)") || !p) return nullptr;
	__atomic_store_n(&g_scratch[device], p, __ATOMIC_RELEASE);
	return p;
}

enum { SP_ARENA, SP_IN, SP_POOL, SP_OUT, SP_NONE };

struct Opnd {
	int space = SP_NONE;
	long off = 0; // SP_ARENA: per-row float offset of the value; others: float offset
	long rs = 0;  // row stride in floats (0 for pool values)
};

enum { ST_BIN, ST_UN, ST_MM, ST_QGEMM, ST_ROW, ST_RED, ST_TRANS, ST_OUTER, ST_TAKE, ST_COPY, ST_SCAN, ST_FILL_STEPS, ST_SSCAN, ST_EW, ST_NOP };

// one member of a merged quantized GEMM: its output and where its columns start
struct QSegOut {
	Opnd o;
	int c0;
	long orr, oj;
};

inline bool same_value(const Opnd &x, const Opnd &y) { return x.space == y.space && x.off == y.off && x.space != SP_NONE; }

// A run of consecutive elementwise instructions over rows of n elements, run
// as one fused launch (tgk_ew). While the program is built, `ops` holds the
// instructions with operands as local ids: j < LOCAL for input j, LOCAL + k
// for the result of op k. finish_ew then keeps a store for each result read
// outside the run, puts the elementwise inputs first and assigns registers.
struct EwStep {
	static constexpr int LOCAL = 1 << 16;
	struct In {
		Opnd o;
		int mode;
		long map;
	};
	struct Op {
		int kind, op, a, b;
		Opnd o;
	};
	int n = 0;
	std::vector<In> in;
	std::vector<Op> ops;
	std::vector<Opnd> out;
	std::vector<tgk_ew_ins> ins;
};

struct Step {
	int kind = 0, op = 0;
	Opnd o, a, b;
	int n = 0, amode = 0, bmode = 0;
	long amap = 0, bmap = 0;
	// generic matmul
	int g = 1, m = 1, k = 1, nn = 1, quant = 0, bits = 0;
	long ag = 0, ai = 0, ap = 0, bg = 0, bp = 0, bj = 0, og = 0, oi = 0, oj = 0;
	long codes = 0, scale = 0; // offsets into the code / scale pools
	// quantized GEMM
	int qw = -1, ni = 1;
	// quantized GEMM: the instructions after it applied in its epilogue (tgk_qgemm_args::epi, rowop;
	// the row op's lines are p0 lines of p1 = C values per batch row)
	struct Epi {
		int kind = 0, op = 0, mode = 0;
		Opnd x;
	};
	int nepi = 0, rowop = 0;
	Epi epi[TGK_EPI_MAX];
	long xr = 0, xj = 0, xk = 0, orr = 0, oc = 0, ojj = 0;
	// row ops, transpose, take
	int p0 = 0, p1 = 0, p2 = 0;
	// copy
	long ooff = 0, aoff = 0;
	int dyn_a = 0, dyn_o = 0;
	// scan
	int T = 0, reverse = 0, body_lo = 0, body_hi = 0, stid = -1;
	// fused selective scan: B and C sequences, A, stacked outputs
	Opnd e0, e1, e2, e3;
	// fused selective scan: neighbours folded in (tgk_sscan_fuse): fdu, du made from dt and b; fgate, the gate's
	// x, D and z in f0, f1, f2 (e3 then holds the gate's output)
	Opnd f0, f1, f2;
	int fdu = 0, fgate = 0;
	// fused elementwise run (index into tg_hip_prog::ews)
	int ew = -1;
	// quantized GEMM whose activation digits the previous step left in the scratch
	int reuse_digits = 0;
	// quantized GEMM: the weight's model value (-1 for a merged weight) and its output segments
	int qv = -1, seg = -1;
};

} // namespace

struct tg_hip_prog {
	tgm_module *m = nullptr;
	int flags = 0, executor = 0, fixed = 0;
	int max_rows = 0;
	hipStream_t st = nullptr;      // stream every launch goes to
	hipStream_t own_st = nullptr;  // the program's own stream (st unless tg_hip_set_stream)
	// pools
	float *d_pool = nullptr;
	int *d_imap = nullptr;
	uint8_t *d_codes = nullptr;
	float *d_fscale = nullptr;
	int *d_qscale = nullptr;
	// layer program
	std::vector<Step> steps;
	std::vector<EwStep> ews;
	std::vector<std::vector<QSegOut>> qsegs; // output segments of merged GEMMs
	std::vector<tgk_qweight> qws;
	long arena_floats = 0; // per row
	float *d_arena = nullptr;
	void *d_scratch = nullptr;
	size_t scratch_bytes = 0;
	Opnd out;
	// row program
	std::vector<rp_ins> rprog;
	rp_ins *d_rprog = nullptr;
	long rp_arena = 0;
	int rp_in_slot = 0, rp_out_ref = 0;
	// calibration capture (tg_hip_quantize_model): value -> capture index, each capture's axis and per-row sample capacity
	std::vector<int> cap_of, cap_axis, cap_rows;
	int cap_both = 0; // a product of two eligible params (both sides would be samples): not captured
	float *d_cap = nullptr;
	long *d_cap_base = nullptr;
	int *d_cap_k = nullptr, *d_cap_rows = nullptr, *d_cap_count = nullptr;
	hipModule_t rp_mod = nullptr;  // the row program compiled for this model
	hipFunction_t rp_fn = nullptr; // its kernel (null: the interpreter runs the program)
	std::string rp_why;            // why the program runs in the interpreter
	// host-buffer batches: a three-slot pipeline (pinned staging, device buffers, copy streams, events)
	static constexpr int NSL = 3; // pipeline slots
	struct HostPipe {
		long chunk = 0;                                            // rows per chunk
		void *h_in[NSL] = {}, *h_out[NSL] = {};                    // pinned staging
		int *h_steps[NSL] = {};
		float *d_in[NSL] = {}, *d_out[NSL] = {};
		int *d_steps[NSL] = {};
		hipStream_t h2d = nullptr, d2h = nullptr;                  // copy streams (default priority)
		hipEvent_t up[NSL] = {}, done[NSL] = {}, down[NSL] = {};   // per slot: copied in, computed, copied out
		hipEvent_t t0[NSL] = {}, t1[NSL] = {};                     // per slot: compute span (timing)
	} hp;
	int *d_steps = nullptr; // steps of tg_hip_batch_device calls that pass none
	// stats
	tg_hip_stats_t stats{};
	hipEvent_t ev0 = nullptr, ev1 = nullptr;
	bool span_open = false; // ev0 marks the first device batch since the last sync
	std::vector<hipEvent_t> tev;
};

namespace {

// ---------------------------------------------------------------- pools ----

struct Pools {
	std::vector<float> f;      // params and constants (f32, or Q16.16 words when fixed)
	std::vector<int> imap;     // broadcast index maps
	std::vector<uint8_t> codes;
	std::vector<float> fscale;
	std::vector<int> qscale;   // Q7.24
	std::vector<long> pool_of; // value -> pool offset, -1 if none
	std::vector<long> codes_of, scale_of;
};

int32_t to_fixed(double v, int frac)
{
	double s = v * (double)(1LL << frac);
	if (s >= 2147483647.0) return INT32_MAX;
	if (s <= -2147483648.0) return INT32_MIN;
	return (int32_t)llround(s);
}

float fixed_word(double v) // a Q16.16 integer stored in a float slot
{
	int32_t q = to_fixed(v, 16);
	float f;
	memcpy(&f, &q, 4);
	return f;
}

long pool_param(Pools &P, const tgm_module *m, int v, bool fixed)
{
	if (P.pool_of[v] >= 0) return P.pool_of[v];
	const tgm_value &x = m->val[v];
	long off = (long)P.f.size();
	for (long i = 0; i < x.n; i++) P.f.push_back(fixed ? fixed_word(x.data[i]) : x.data[i]);
	while (P.f.size() % 16) P.f.push_back(0.0f);
	P.pool_of[v] = off;
	return off;
}

long pool_codes(Pools &P, const tgm_module *m, int v)
{
	if (P.codes_of[v] >= 0) return P.codes_of[v];
	const tgm_value &x = m->val[v];
	long off = (long)P.codes.size(), nb = x.qbits == 8 ? x.n : (x.n + 1) / 2;
	P.codes.insert(P.codes.end(), x.q, x.q + nb);
	while (P.codes.size() % 16) P.codes.push_back(0);
	int nch = x.sh.dim[x.qaxis];
	P.scale_of[v] = (long)P.fscale.size();
	for (int i = 0; i < nch; i++) {
		P.fscale.push_back(x.qs[i]);
		P.qscale.push_back(to_fixed(x.qs[i], 24));
	}
	P.codes_of[v] = off;
	return off;
}

// ------------------------------------------------------- shape helpers ----

long numel(const tgm_shape &s) { return tgm_numel(&s); }

void matmul_dims(const tgm_shape &a, const tgm_shape &b, int &m, int &k, int &n, int &g)
{
	g = a.rank == 3 && b.rank == 3 ? a.dim[0] : 1;
	m = a.rank == 3 ? (g > 1 || b.rank == 3 ? a.dim[1] : a.dim[0] * a.dim[1]) : a.rank == 2 ? a.dim[0] : 1;
	k = a.dim[a.rank - 1];
	n = b.rank >= 2 ? b.dim[b.rank - 1] : 1;
}

// which axis a param needs as operand of a matmul (src/ops.c:310-320)
int q_axis_for(const tgm_module *m, int v, const tgm_ins &in)
{
	if (m->val[v].sh.rank != 2 || in.op != TGM_MATMUL) return -1;
	if (in.a[0] == v && in.a[1] != v) return 0;
	if (in.a[1] == v && in.a[0] != v) return 1;
	return -1;
}

// Broadcast index maps: for every output element, the element of each operand
// it reads (NumPy broadcasting, dimensions aligned from the right), or mode 0
// (same element) / 1 (the single element) when no map is needed.
void bcast(const tgm_shape &so, const tgm_shape &sa, std::vector<int> &imap, int &mode, long &mapoff)
{
	long n = numel(so), na = numel(sa);
	mapoff = 0;
	if (na == n) {
		mode = 0;
		return;
	}
	if (na == 1) {
		mode = 1;
		return;
	}
	mode = 2;
	mapoff = (long)imap.size();
	int r = so.rank, idx[TGM_MAXRANK] = { 0 };
	long st[TGM_MAXRANK], acc = 1;
	for (int i = r - 1; i >= 0; i--) {
		int j = i - (r - sa.rank), d = j >= 0 ? sa.dim[j] : 1;
		st[i] = d == 1 ? 0 : acc;
		acc *= d;
	}
	for (long e = 0; e < n; e++) {
		long ia = 0;
		for (int i = 0; i < r; i++) ia += idx[i] * st[i];
		imap.push_back((int)ia);
		for (int i = r - 1; i >= 0; i--) {
			if (++idx[i] < so.dim[i]) break;
			idx[i] = 0;
		}
	}
}

bool has_think(const tgm_block *b)
{
	for (int i = 0; i < b->len; i++) {
		if (b->v[i].op == TGM_THINK) return true;
		if (b->v[i].body && has_think(b->v[i].body)) return true;
	}
	return false;
}

// ------------------------------------------------------ layer program ----

struct LB {
	tg_hip_prog *p;
	tgm_module *m;
	Pools P;
	std::vector<Opnd> where; // value -> operand
	std::vector<char> loopw; // values written in place by loops (scan carries, slices, stacks)
	std::vector<int> tview;  // rank-2 transposes read only by one f32 matmul: the transposed value (else -1)
	std::vector<char> skip;  // top-block instructions folded into a fused scan (plan_sscan)
	struct SscanPlan {
		int dux = -1;                       // du = mul(dt, dux): the kernel forms it
		int gx = -1, gD = -1, gz = -1, out = -1; // out = (ys + gx * gD) * silu(gz): the kernel writes it
	};
	std::map<const tgm_ins *, SscanPlan> sscan;
	std::map<int, int> lone; // top-block quantized product -> the lone activation its stores apply (plan_lone_acts)
};

void count_uses(const tgm_block *b, std::vector<int> &u);

// A rank-2 transpose whose only reader is an unquantized rank-2 matmul of the
// top block is not materialised: the matmul reads the transpose's input with
// its strides swapped (same elements, same products, same order).
void mark_transpose_views(LB &L)
{
	const tgm_module *m = L.m;
	L.tview.assign((size_t)m->nval, -1);
	std::vector<int> uses((size_t)m->nval, 0);
	count_uses(&m->top, uses);
	uses[(size_t)m->output]++;
	const tgm_block &b = m->top;
	std::vector<int> src((size_t)m->nval, -1);
	for (int i = 0; i < b.len; i++) {
		const tgm_ins &in = b.v[i];
		if (in.op == TGM_TRANSPOSE && m->val[in.a[0]].sh.rank == 2 && uses[(size_t)in.out] == 1) src[(size_t)in.out] = in.a[0];
		if (in.op != TGM_MATMUL) continue;
		const tgm_value &va = m->val[in.a[0]], &vb = m->val[in.a[1]];
		if (va.sh.rank != 2 || vb.sh.rank != 2 || va.qbits || vb.qbits || in.a[0] == in.a[1]) continue;
		for (int j = 0; j < 2; j++)
			if (src[(size_t)in.a[j]] >= 0) L.tview[(size_t)in.a[j]] = src[(size_t)in.a[j]];
	}
}

Opnd value_opnd(LB &L, int v)
{
	Opnd &w = L.where[v];
	if (w.space != SP_NONE) return w;
	const tgm_value &x = L.m->val[v];
	if (x.kind == TGM_PARAM || x.kind == TGM_STATE) {
		w.space = SP_POOL;
		w.off = pool_param(L.P, L.m, v, false);
		w.rs = 0;
	} else if (x.kind == TGM_INPUT) {
		w.space = SP_IN;
		w.off = x.in_off;
		w.rs = L.m->per;
	} else {
		w.space = SP_ARENA;
		w.off = v; // the value's id until place_arena assigns its offset
		w.rs = x.n;
	}
	return w;
}

// Arena placement by lifetime. Every arena operand of a step names its value
// (Opnd::off holds the value id while the steps are built). A value lives from
// the first to the last step that names it, both included, so a step's output
// never shares memory with its inputs. A value whose lifetime crosses the
// boundary of a scan body (read inside but made outside, a carry, a stacked
// output) lives for the whole scan, since the body runs T times; values made
// and used within one pass of a body stay local to it. Offsets are then
// assigned in order of first use, best fit among the blocks freed so far.
void place_arena(tg_hip_prog *p, const tgm_module *m)
{
	auto &S = p->steps;
	const int nv = m->nval;
	std::vector<long> first(nv, -1), last(nv, -1);
	auto touch = [&](const Opnd &o, long i) {
		if (o.space != SP_ARENA) return;
		const int v = (int)o.off;
		if (first[v] < 0) first[v] = i;
		if (i > last[v]) last[v] = i;
		if (i < first[v]) first[v] = i;
	};
	for (long i = 0; i < (long)S.size(); i++) {
		const Step &st = S[i];
		for (const Opnd *o : { &st.o, &st.a, &st.b, &st.e0, &st.e1, &st.e2, &st.e3, &st.f0, &st.f1, &st.f2 }) touch(*o, i);
		for (int e = 0; e < st.nepi; e++) touch(st.epi[e].x, i);
		if (st.kind == ST_EW) {
			for (const EwStep::In &x : p->ews[(size_t)st.ew].in) touch(x.o, i);
			for (const Opnd &x : p->ews[(size_t)st.ew].out) touch(x, i);
		}
		if (st.kind == ST_QGEMM && st.seg >= 0)
			for (const QSegOut &x : p->qsegs[(size_t)st.seg]) touch(x.o, i);
	}
	touch(p->out, (long)S.size());
	// scans, innermost first (shorter ranges are nested in longer ones)
	std::vector<std::pair<long, long>> scans;
	for (long i = 0; i < (long)S.size(); i++)
		if (S[i].kind == ST_SCAN) scans.push_back({ i, (long)S[i].body_hi - 1 });
	std::sort(scans.begin(), scans.end(), [](const std::pair<long, long> &x, const std::pair<long, long> &y) {
		return x.second - x.first < y.second - y.first;
	});
	for (auto &sc : scans)
		for (int v = 0; v < nv; v++) {
			if (first[v] < 0 || last[v] < sc.first || first[v] > sc.second) continue; // disjoint
			if (first[v] > sc.first && last[v] <= sc.second) continue;                 // local to the body
			first[v] = std::min(first[v], sc.first);
			last[v] = std::max(last[v], sc.second);
		}
	std::vector<int> order;
	for (int v = 0; v < nv; v++)
		if (first[v] >= 0) order.push_back(v);
	std::sort(order.begin(), order.end(), [&](int x, int y) { return first[x] < first[y] || (first[x] == first[y] && x < y); });
	std::vector<long> off(nv, -1);
	std::vector<std::pair<long, long>> freel; // (offset, size) blocks
	std::vector<int> live;
	long end = 0;
	for (int v : order) {
		for (size_t j = 0; j < live.size();) { // free what ended before v begins
			const int u = live[j];
			if (last[u] < first[v]) {
				freel.push_back({ off[u], (m->val[u].n + 63) / 64 * 64 });
				live[j] = live.back();
				live.pop_back();
			} else
				j++;
		}
		std::sort(freel.begin(), freel.end());
		for (size_t j = 0; j + 1 < freel.size();) { // merge neighbours
			if (freel[j].first + freel[j].second == freel[j + 1].first) {
				freel[j].second += freel[j + 1].second;
				freel.erase(freel.begin() + (long)j + 1);
			} else
				j++;
		}
		const long need = (m->val[v].n + 63) / 64 * 64;
		long best = -1;
		for (size_t j = 0; j < freel.size(); j++)
			if (freel[j].second >= need && (best < 0 || freel[j].second < freel[(size_t)best].second)) best = (long)j;
		if (best >= 0) {
			off[v] = freel[(size_t)best].first;
			freel[(size_t)best].first += need;
			freel[(size_t)best].second -= need;
			if (!freel[(size_t)best].second) freel.erase(freel.begin() + best);
		} else if (!freel.empty() && freel.back().first + freel.back().second == end) { // grow the last free block
			off[v] = freel.back().first;
			end = off[v] + need;
			freel.pop_back();
		} else {
			off[v] = end;
			end += need;
		}
		live.push_back(v);
	}
	auto fix = [&](Opnd &o) {
		if (o.space == SP_ARENA) o.off = off[(int)o.off];
	};
	for (Step &st : S) {
		for (Opnd *o : { &st.o, &st.a, &st.b, &st.e0, &st.e1, &st.e2, &st.e3, &st.f0, &st.f1, &st.f2 }) fix(*o);
		for (int e = 0; e < st.nepi; e++) fix(st.epi[e].x);
	}
	for (EwStep &E : p->ews) {
		for (EwStep::In &x : E.in) fix(x.o);
		for (Opnd &x : E.out) fix(x);
	}
	for (auto &g : p->qsegs)
		for (QSegOut &x : g) fix(x.o);
	fix(p->out);
	p->arena_floats = end;
}

bool layer_block(LB &L, const tgm_block *b);

// Operand shape sa broadcast to so by repeating it whole (sa, leading 1s
// dropped, is a suffix of so): element e reads e mod numel(sa). Such operands
// take mode 3 (period numel(sa)) instead of an index map.
bool suffix_broadcast(const tgm_shape &so, const tgm_shape &sa)
{
	int lo = 0;
	while (lo < sa.rank && sa.dim[lo] == 1) lo++;
	const int ra = sa.rank - lo;
	if (ra > so.rank) return false;
	for (int i = 0; i < ra; i++)
		if (sa.dim[lo + i] != so.dim[so.rank - ra + i]) return false;
	return true;
}

// Adds one elementwise instruction, to the fused run the previous step holds
// when it can (same row length, room left, operands that the run computed
// read elementwise), else to a new run. The run's inputs plus its results
// never exceed the kernel's register file, so every run has registers.
void ew_append(LB &L, int kind, int op, const Opnd &a, int amode, long amap, const Opnd &b, int bmode, long bmap, const Opnd &o, int n)
{
	auto &S = L.p->steps;
	auto local = [](const EwStep &E, const Opnd &x) {
		for (size_t k = 0; k < E.ops.size(); k++)
			if (same_value(E.ops[k].o, x)) return (int)k;
		return -1;
	};
	auto input = [](const EwStep &E, const Opnd &x, int mode, long map) {
		for (size_t j = 0; j < E.in.size(); j++)
			if (same_value(E.in[j].o, x) && E.in[j].o.rs == x.rs && E.in[j].mode == mode && E.in[j].map == map)
				return (int)j;
		return -1;
	};
	const int nops = kind == TGK_EW_BIN ? 2 : 1;
	const Opnd *opd[2] = { &a, &b };
	const int mode[2] = { amode, bmode };
	const long map[2] = { amap, bmap };
	bool fits = !S.empty() && S.back().kind == ST_EW;
	if (fits) {
		const EwStep &E = L.p->ews[(size_t)S.back().ew];
		int new_in = 0;
		for (int j = 0; j < nops; j++) {
			const int k = local(E, *opd[j]);
			if (k >= 0 && mode[j] != 0) fits = false;
			if (k < 0 && input(E, *opd[j], mode[j], map[j]) < 0 && !(j == 1 && same_value(a, b) && a.rs == b.rs && amode == bmode && amap == bmap))
				new_in++;
		}
		fits = fits && E.n == n && (int)E.in.size() + new_in <= TGK_EW_MAXIN &&
		       (int)(E.in.size() + new_in + E.ops.size() + 1) <= TGK_EW_REGS && (int)E.ops.size() < TGK_EW_MAXOUT;
	}
	if (!fits) {
		Step st;
		st.kind = ST_EW;
		st.ew = (int)L.p->ews.size();
		L.p->ews.emplace_back();
		L.p->ews.back().n = n;
		S.push_back(st);
	}
	EwStep &E = L.p->ews[(size_t)S.back().ew];
	int id[2] = { 0, 0 };
	for (int j = 0; j < nops; j++) {
		const int k = local(E, *opd[j]);
		if (k >= 0) {
			id[j] = EwStep::LOCAL + k;
			continue;
		}
		int q = input(E, *opd[j], mode[j], map[j]);
		if (q < 0) {
			E.in.push_back({ *opd[j], mode[j], map[j] });
			q = (int)E.in.size() - 1;
		}
		id[j] = q;
	}
	E.ops.push_back({ kind, op, id[0], id[1], o });
}

// Completes every fused run once all steps exist: which results are read
// outside their run (they are stored, the others live only in registers),
// elementwise inputs first, registers by lifetime.
void finish_ew(tg_hip_prog *p)
{
	std::vector<Opnd> used; // operands read or written by steps other than fused runs, plus the output
	for (const Step &st : p->steps)
		if (st.kind != ST_EW && st.kind != ST_NOP) {
			for (const Opnd *o : { &st.o, &st.a, &st.b, &st.e0, &st.e1, &st.e2, &st.e3, &st.f0, &st.f1, &st.f2 })
				if (o->space == SP_ARENA || o->space == SP_OUT) used.push_back(*o);
			for (int e = 0; e < st.nepi; e++) // a GEMM epilogue's operands
				if (st.epi[e].x.space == SP_ARENA || st.epi[e].x.space == SP_OUT) used.push_back(st.epi[e].x);
		}
	for (const auto &g : p->qsegs)
		for (const QSegOut &x : g) used.push_back(x.o);
	for (const EwStep &E : p->ews)
		for (const EwStep::In &x : E.in) used.push_back(x.o);
	used.push_back(p->out);
	auto read_outside = [&](const Opnd &o) {
		if (o.space == SP_OUT) return true;
		for (const Opnd &u : used)
			if (same_value(u, o)) return true;
		return false;
	};
	for (Step &st : p->steps) { // a run of one instruction takes the specialised kernel
		if (st.kind != ST_EW || p->ews[(size_t)st.ew].ops.size() != 1) continue;
		EwStep &E = p->ews[(size_t)st.ew];
		const EwStep::Op &q = E.ops[0];
		st.kind = q.kind == TGK_EW_BIN ? ST_BIN : ST_UN;
		st.op = q.op;
		st.n = E.n;
		st.o = q.o;
		st.a = E.in[(size_t)q.a].o;
		st.amode = E.in[(size_t)q.a].mode;
		st.amap = E.in[(size_t)q.a].map;
		if (q.kind == TGK_EW_BIN) {
			st.b = E.in[(size_t)q.b].o;
			st.bmode = E.in[(size_t)q.b].mode;
			st.bmap = E.in[(size_t)q.b].map;
		}
		st.ew = -1;
		E = EwStep{};
	}
	for (EwStep &E : p->ews) {
		if (E.ops.empty()) continue;
		const int nin = (int)E.in.size(), nop = (int)E.ops.size();
		// elementwise inputs first, then whole-row repeats of a multiple of 4
		// elements (both load as float4), then the rest
		std::vector<int> order, pos(nin);
		auto cls = [&](int j) {
			return E.in[j].mode == 0 ? 0 : E.in[j].mode == 3 && E.in[j].map % 4 == 0 && E.n / E.in[j].map < (1 << 22) ? 1 : 2;
		};
		for (int c = 0; c < 3; c++)
			for (int j = 0; j < nin; j++)
				if (cls(j) == c) order.push_back(j);
		std::vector<EwStep::In> in2;
		for (int j = 0; j < nin; j++) {
			pos[order[j]] = j;
			in2.push_back(E.in[order[j]]);
		}
		E.in = in2;
		// local values densely: input j is j, the result of op k is nin + k
		auto dense = [&](int id) { return id < EwStep::LOCAL ? pos[id] : nin + (id - EwStep::LOCAL); };
		std::vector<int> lastd(nin + nop, -1); // last op reading each value
		for (int k = 0; k < nop; k++) {
			const EwStep::Op &q = E.ops[k];
			lastd[dense(q.a)] = k;
			if (q.kind == TGK_EW_BIN) lastd[dense(q.b)] = k;
		}
		// Linearise for the accumulator machine. A value leaves the accumulator
		// for a register (SAVE) only when it is read again later; inputs start
		// in registers 0 .. nin - 1. The append limits (inputs + ops within the
		// register file) guarantee a free register whenever one is needed.
		std::vector<int> rg(nin + nop, -1), busy(TGK_EW_REGS, 0);
		for (int j = 0; j < nin; j++) rg[j] = j, busy[j] = 1;
		int acc = -1;
		E.ins.clear();
		E.out.clear();
		auto keep = [&](int v) { // v (in the accumulator) is read again after this op: give it a register
			if (rg[v] >= 0) return;
			int r = 0;
			while (busy[r]) r++;
			busy[r] = 1;
			rg[v] = r;
			E.ins.push_back({ TGK_EW_SAVE, 0, r, 0, 0 });
		};
		for (int k = 0; k < nop; k++) {
			for (int v = 0; v < nin + nop; v++) // registers of values no longer read
				if (rg[v] >= 0 && lastd[v] < k) busy[rg[v]] = 0, rg[v] = -1;
			const EwStep::Op &q = E.ops[k];
			const int a = dense(q.a), b = q.kind == TGK_EW_BIN ? dense(q.b) : -1;
			if (q.kind == TGK_EW_UN || (a != acc && b != acc)) { // the first operand goes to the accumulator
				if (a != acc) {
					if (acc >= 0 && lastd[acc] >= k) keep(acc);
					E.ins.push_back({ TGK_EW_LOAD, 0, 0, rg[a], 0 });
					acc = a;
				}
				if (lastd[a] > k || (b == a)) keep(a);
				if (q.kind == TGK_EW_UN) E.ins.push_back({ TGK_EW_UN, q.op, 0, 0, 0 });
				else E.ins.push_back({ TGK_EW_BIN, q.op, 0, rg[b], 0 });
			} else if (a == acc) { // acc = acc op b
				if (lastd[a] > k || b == a) keep(a);
				E.ins.push_back({ TGK_EW_BIN, q.op, 0, rg[b], 0 });
			} else { // b in the accumulator: acc = a op acc
				if (lastd[b] > k) keep(b);
				E.ins.push_back({ TGK_EW_BINR, q.op, 0, rg[a], 0 });
			}
			acc = nin + k;
			if (read_outside(q.o)) {
				E.ins.push_back({ TGK_EW_STORE, 0, (int)E.out.size(), 0, 0 });
				E.out.push_back(q.o);
			}
		}
	}
}

// A scan whose body is exactly the selective-state-space recurrence
//   (x0 [D 1] (reshape dt)) (x1 [D N] (mul x0 A)) (x2 (exp x1)) (x3 (mul x2 h))
//   (x4 (outer du B)) (x5 (add x3 x4)) (y [D] (matmul x5 C)), next h = x5, emit y
// (dt, du [D] and B, C [N] the scan's four sequence slices, A a [D N] param,
// h the only carry; commuted mul/add operands accepted) runs as one fused
// kernel (tgk_sscan) instead of seven launches per step. Any other body takes
// the general path.
bool sscan_shape(const tgm_module *m, const tgm_ins &in, int &jdt, int &jdu, int &jb, int &jc, int &A)
{
	if (in.op != TGM_SCAN || in.nc != 1 || in.ny != 1 || in.nx != 4 || in.stid >= 0 || !in.body || in.body->len != 7) return false;
	const tgm_ins *b = in.body->v;
	const int h = in.c[0];
	const tgm_shape &hs = m->val[h].sh;
	if (hs.rank != 2) return false;
	const int D = hs.dim[0], N = hs.dim[1];
	if (!tgk_sscan_supported(N)) return false;
	auto slice = [&](int v) {
		for (int j = 0; j < in.nx; j++)
			if (in.xt[j] == v) return j;
		return -1;
	};
	auto shaped = [&](int v, int rank, int d0, int d1) {
		const tgm_shape &x = m->val[v].sh;
		return x.rank == rank && x.dim[0] == d0 && (rank < 2 || x.dim[1] == d1);
	};
	auto pair = [](const tgm_ins &i, int u, int v) { return (i.a[0] == u && i.a[1] == v) || (i.a[0] == v && i.a[1] == u); };
	if (b[0].op != TGM_RESHAPE || !shaped(b[0].out, 2, D, 1) || !shaped(b[0].a[0], 1, D, 0)) return false;
	jdt = slice(b[0].a[0]);
	if (b[1].op != TGM_MUL || !shaped(b[1].out, 2, D, N)) return false;
	A = b[1].a[0] == b[0].out ? b[1].a[1] : b[1].a[1] == b[0].out ? b[1].a[0] : -1;
	if (A < 0 || m->val[A].kind != TGM_PARAM || m->val[A].qbits || !shaped(A, 2, D, N)) return false;
	if (b[2].op != TGM_EXP || b[2].a[0] != b[1].out) return false;
	if (b[3].op != TGM_MUL || !pair(b[3], b[2].out, h)) return false;
	if (b[4].op != TGM_OUTER || !shaped(b[4].a[0], 1, D, 0) || !shaped(b[4].a[1], 1, N, 0)) return false;
	jdu = slice(b[4].a[0]), jb = slice(b[4].a[1]);
	if (b[5].op != TGM_ADD || !pair(b[5], b[3].out, b[4].out)) return false;
	if (b[6].op != TGM_MATMUL || b[6].a[0] != b[5].out || !shaped(b[6].out, 1, D, 0) || !shaped(b[6].a[1], 1, N, 0)) return false;
	jc = slice(b[6].a[1]);
	if (jdt < 0 || jdu < 0 || jb < 0 || jc < 0) return false;
	if (jdt == jdu || jdt == jb || jdt == jc || jdu == jb || jdu == jc || jb == jc) return false;
	return in.cnext[0] == b[5].out && in.y[0] == b[6].out;
}

// A fused scan of the top block takes in what Mamba's block computes right
// around it, when nothing else reads the values in between (every value is
// written once, so they can be formed where they are read):
//  - its du sequence made by (mul dt X), dt its own dt sequence, X of du's
//    shape: the kernel forms dt_t * X_t as it loads the steps;
//  - its stacked output read only by (add ys P) with P = (mul X2 Dv), Dv a
//    rank-1 param of one value per channel, whose sum is read only by
//    (mul S G), G = (silu Z): the kernel writes (ys + X2 Dv) * silu(Z) in
//    place of ys. X2 and Z must be made before the scan.
// The folded instructions are skipped by layer_block; each operation is the
// one their kernels compute, so the values are unchanged.
void plan_sscan(LB &L)
{
	const tgm_module *m = L.m;
	const tgm_block &b = m->top;
	L.skip.assign((size_t)b.len, 0);
	std::vector<int> uses((size_t)m->nval, 0), prod((size_t)m->nval, -1), reader((size_t)m->nval, -1);
	count_uses(&b, uses);
	uses[(size_t)m->output]++;
	for (int i = 0; i < b.len; i++) {
		const tgm_ins &in = b.v[i];
		if (in.out >= 0) prod[(size_t)in.out] = i;
		for (int j = 0; j < in.na; j++) reader[(size_t)in.a[j]] = i;
		if (in.op == TGM_SCAN) {
			for (int k = 0; k < in.ny; k++) prod[(size_t)in.ys[k]] = i;
			for (int k = 0; k < in.nx; k++) reader[(size_t)in.x[k]] = i;
			for (int k = 0; k < in.nc; k++) reader[(size_t)in.cinit[k]] = i;
		}
	}
	auto same_shape = [&](int u, int v) {
		const tgm_shape &x = m->val[u].sh, &y = m->val[v].sh;
		if (x.rank != y.rank) return false;
		for (int d = 0; d < x.rank; d++)
			if (x.dim[d] != y.dim[d]) return false;
		return true;
	};
	auto other = [](const tgm_ins &in, int v) { return in.na != 2 ? -1 : in.a[0] == v ? in.a[1] : in.a[1] == v ? in.a[0] : -1; };
	auto before = [&](int v, int i) { return prod[(size_t)v] < i; }; // made before instruction i (or not made here at all)
	for (int i = 0; i < b.len; i++) {
		const tgm_ins &in = b.v[i];
		int jdt, jdu, jb, jc, A;
		if (!sscan_shape(m, in, jdt, jdu, jb, jc, A)) continue;
		LB::SscanPlan plan;
		const int du = in.x[jdu], dt = in.x[jdt], j = prod[(size_t)du];
		if (j >= 0 && j < i && uses[(size_t)du] == 1 && !L.loopw[(size_t)du] && b.v[j].op == TGM_MUL) {
			const int X = other(b.v[j], dt);
			if (X >= 0 && X != dt && same_shape(X, du) && before(X, j)) {
				plan.dux = X;
				L.skip[(size_t)j] = 1;
			}
		}
		const int ys = in.ys[0], D = m->val[in.c[0]].sh.dim[0];
		const int k1 = reader[(size_t)ys];
		if (uses[(size_t)ys] == 1 && k1 > i && b.v[k1].op == TGM_ADD) {
			const int P = other(b.v[k1], ys), k0 = P >= 0 ? prod[(size_t)P] : -1;
			const int S = b.v[k1].out, k3 = reader[(size_t)S];
			if (k0 >= 0 && uses[(size_t)P] == 1 && b.v[k0].op == TGM_MUL && same_shape(P, ys) && uses[(size_t)S] == 1 && k3 > k1 &&
			    b.v[k3].op == TGM_MUL && same_shape(S, ys)) {
				int X2 = -1, Dv = -1;
				for (int q = 0; q < 2; q++) {
					const int u = b.v[k0].a[q], v = b.v[k0].a[1 - q];
					const tgm_value &pv = m->val[(size_t)v];
					if (pv.kind == TGM_PARAM && !pv.qbits && pv.sh.rank == 1 && pv.sh.dim[0] == D && same_shape(u, ys)) X2 = u, Dv = v;
				}
				const int G = other(b.v[k3], S), k2 = G >= 0 ? prod[(size_t)G] : -1;
				const int Z = k2 >= 0 && b.v[k2].op == TGM_SILU ? b.v[k2].a[0] : -1;
				if (X2 >= 0 && before(X2, i) && Z >= 0 && uses[(size_t)G] == 1 && same_shape(G, ys) && same_shape(Z, ys) && before(Z, i) &&
				    k2 != j && k0 != j) {
					plan.gx = X2, plan.gD = Dv, plan.gz = Z, plan.out = b.v[k3].out;
					L.skip[(size_t)k0] = L.skip[(size_t)k1] = L.skip[(size_t)k2] = L.skip[(size_t)k3] = 1;
				}
			}
		}
		if (plan.dux >= 0 || plan.out >= 0) L.sscan[&in] = plan;
	}
	for (char k : L.skip) L.p->stats.scan_folded_ins += k;
}

bool match_sscan(LB &L, const tgm_ins &in, Step &st)
{
	const tgm_module *m = L.m;
	int jdt, jdu, jb, jc, A;
	if (!sscan_shape(m, in, jdt, jdu, jb, jc, A)) return false;
	const int h = in.c[0];
	const tgm_shape &hs = m->val[h].sh;
	const int D = hs.dim[0], N = hs.dim[1];
	const auto pl = L.sscan.find(&in);
	const LB::SscanPlan plan = pl == L.sscan.end() ? LB::SscanPlan{} : pl->second;
	st.kind = ST_SSCAN;
	st.o = value_opnd(L, h);
	st.a = value_opnd(L, in.x[jdt]);
	st.fdu = plan.dux >= 0;
	st.b = value_opnd(L, st.fdu ? plan.dux : in.x[jdu]);
	st.e0 = value_opnd(L, in.x[jb]);
	st.e1 = value_opnd(L, in.x[jc]);
	st.e2 = value_opnd(L, A);
	st.fgate = plan.out >= 0;
	if (st.fgate) {
		st.f0 = value_opnd(L, plan.gx);
		st.f1 = value_opnd(L, plan.gD);
		st.f2 = value_opnd(L, plan.gz);
	}
	st.e3 = value_opnd(L, st.fgate ? plan.out : in.ys[0]);
	st.p0 = D;
	st.p1 = N;
	st.T = in.T;
	st.reverse = in.reverse;
	return true;
}

// which operand of a matmul is a quantized parameter read along its channel
// axis (1: a, 2: b), 0 when none: those products run as quantized GEMMs
int matmul_quant(const tgm_module *m, const tgm_ins &in)
{
	const tgm_value &va = m->val[in.a[0]], &vb = m->val[in.a[1]];
	int mm, kk, nn, gg;
	matmul_dims(va.sh, vb.sh, mm, kk, nn, gg);
	if (gg == 1 && va.qbits && q_axis_for(m, in.a[0], in) == va.qaxis) return 1;
	if (gg == 1 && vb.qbits && q_axis_for(m, in.a[1], in) == vb.qaxis) return 2;
	return 0;
}

bool layer_ins(LB &L, const tgm_ins &in)
{
	tgm_module *m = L.m;
	auto &S = L.p->steps;
	Step s;
	switch (in.op) {
	case TGM_CONST: {
		long off = (long)L.P.f.size();
		L.P.f.push_back(in.k);
		while (L.P.f.size() % 16) L.P.f.push_back(0.0f);
		Opnd &w = L.where[in.out];
		w.space = SP_POOL;
		w.off = off;
		w.rs = 0;
		return true;
	}
	case TGM_RESHAPE: {
		Opnd a = value_opnd(L, in.a[0]);
		if (!L.loopw[in.a[0]] && !L.loopw[in.out]) { // same elements, new shape: share the operand
			L.where[in.out] = a;
			return true;
		}
		s.kind = ST_COPY;
		s.o = value_opnd(L, in.out);
		s.a = a;
		s.n = (int)m->val[in.out].n;
		break;
	}
	case TGM_ADD: case TGM_SUB: case TGM_MUL: case TGM_DIV: case TGM_MAX: case TGM_MIN: {
		int amode, bmode;
		long amap, bmap;
		bcast(m->val[in.out].sh, m->val[in.a[0]].sh, L.P.imap, amode, amap);
		if (amode == 2 && suffix_broadcast(m->val[in.out].sh, m->val[in.a[0]].sh)) {
			L.P.imap.resize((size_t)amap); // the map just added is not needed
			amode = 3;
			amap = m->val[in.a[0]].n;
		}
		bcast(m->val[in.out].sh, m->val[in.a[1]].sh, L.P.imap, bmode, bmap);
		if (bmode == 2 && suffix_broadcast(m->val[in.out].sh, m->val[in.a[1]].sh)) {
			L.P.imap.resize((size_t)bmap);
			bmode = 3;
			bmap = m->val[in.a[1]].n;
		}
		ew_append(L, TGK_EW_BIN, in.op - TGM_ADD, value_opnd(L, in.a[0]), amode, amap, value_opnd(L, in.a[1]), bmode, bmap,
			  value_opnd(L, in.out), (int)m->val[in.out].n);
		return true;
	}
	case TGM_NEG: case TGM_TANH: case TGM_RELU: case TGM_SIGMOID: case TGM_EXP: case TGM_SQRT: case TGM_GELU:
	case TGM_SILU: case TGM_SOFTPLUS: case TGM_LOG: case TGM_SIN: case TGM_COS: case TGM_FLOOR: case TGM_STEP:
		ew_append(L, TGK_EW_UN, in.op, value_opnd(L, in.a[0]), 0, 0, Opnd{}, 0, 0, value_opnd(L, in.out),
			  (int)m->val[in.out].n);
		return true;
	case TGM_MATMUL: {
		const tgm_value &va = m->val[in.a[0]], &vb = m->val[in.a[1]];
		int mm, kk, nn, gg;
		matmul_dims(va.sh, vb.sh, mm, kk, nn, gg);
		const int quant = matmul_quant(m, in);
		s.o = value_opnd(L, in.out);
		if (quant && !(L.p->flags & TG_HIP_EXACT)) {
			const tgm_value &w = quant == 1 ? va : vb;
			int v = quant == 1 ? in.a[0] : in.a[1];
			Opnd x = value_opnd(L, quant == 1 ? in.a[1] : in.a[0]);
			tgk_qweight qw; // packed once every step exists (GEMMs on the same activations are merged first)
			memset(&qw, 0, sizeof qw);
			int C = w.sh.dim[w.qaxis], K = w.sh.dim[1 - w.qaxis];
			qw.C = C, qw.K = K, qw.bits = w.qbits, qw.axis = w.qaxis;
			qw.Kp = (K + 63) / 64 * 64, qw.Cp = (C + 255) / 256 * 256;
			L.p->qws.push_back(qw);
			s.kind = ST_QGEMM;
			s.qw = (int)L.p->qws.size() - 1;
			s.qv = v;
			s.a = x;
			if (quant == 1) { // W[C][K] @ x[K][n]: rows (r, j), element k at k*n
				s.ni = nn;
				s.xr = x.rs, s.xj = 1, s.xk = nn;
				s.orr = s.o.rs, s.oc = nn, s.ojj = 1;
			} else { // x[m][K] @ W[K][C]: rows (r, i), element k at i*K + k
				s.ni = mm;
				s.xr = x.rs, s.xj = kk, s.xk = 1;
				s.orr = s.o.rs, s.oc = 1, s.ojj = nn;
			}
			size_t need = tgk_qgemm_scratch(L.p->max_rows * s.ni, qw.Kp);
			if (need > L.p->scratch_bytes) L.p->scratch_bytes = need;
			L.p->stats.macs += (double)C * K * s.ni;
			break;
		}
		s.kind = ST_MM;
		s.g = gg, s.m = mm, s.k = kk, s.nn = nn, s.quant = quant;
		s.a = quant == 1 ? Opnd{ SP_NONE, 0, 0 } : value_opnd(L, in.a[0]);
		s.b = quant == 2 ? Opnd{ SP_NONE, 0, 0 } : value_opnd(L, in.a[1]);
		if (quant == 1) s.b = value_opnd(L, in.a[1]);
		if (quant == 2) s.a = value_opnd(L, in.a[0]);
		s.ag = (long)mm * kk, s.ai = kk, s.ap = 1;
		s.bg = (long)kk * nn, s.bp = nn, s.bj = 1;
		s.og = (long)mm * nn, s.oi = nn, s.oj = 1;
		if (!quant && L.tview[(size_t)in.a[0]] >= 0) { // A = transpose(X), X [k m]: A[i][p] = X[p][i]
			s.a = value_opnd(L, L.tview[(size_t)in.a[0]]);
			s.ai = 1, s.ap = mm;
		}
		if (!quant && L.tview[(size_t)in.a[1]] >= 0) { // B = transpose(Y), Y [n k]: B[p][j] = Y[j][p]
			s.b = value_opnd(L, L.tview[(size_t)in.a[1]]);
			s.bp = 1, s.bj = kk;
		}
		if (quant) {
			int v = quant == 1 ? in.a[0] : in.a[1];
			s.bits = m->val[v].qbits;
			s.codes = pool_codes(L.P, m, v);
			s.scale = L.P.scale_of[v];
			L.p->stats.macs += (double)mm * kk * nn;
		}
		break;
	}
	case TGM_SOFTMAX: case TGM_RMSNORM: {
		const tgm_shape &sa = m->val[in.a[0]].sh;
		s.kind = ST_ROW;
		s.op = in.op;
		s.a = value_opnd(L, in.a[0]);
		s.o = value_opnd(L, in.out);
		s.p1 = sa.rank ? sa.dim[sa.rank - 1] : 1;
		s.p0 = (int)(numel(sa) / s.p1);
		break;
	}
	case TGM_SUM: case TGM_MEAN:
		s.kind = ST_RED;
		s.op = in.op;
		s.a = value_opnd(L, in.a[0]);
		s.o = value_opnd(L, in.out);
		s.n = (int)m->val[in.a[0]].n;
		break;
	case TGM_TRANSPOSE: {
		if (L.tview[(size_t)in.out] >= 0) return true; // read in place by its matmul
		const tgm_shape &sa = m->val[in.a[0]].sh;
		s.kind = ST_TRANS;
		s.a = value_opnd(L, in.a[0]);
		s.o = value_opnd(L, in.out);
		s.p0 = sa.rank == 3 ? sa.dim[0] : 1;
		s.p1 = sa.dim[sa.rank - 2];
		s.p2 = sa.dim[sa.rank - 1];
		break;
	}
	case TGM_OUTER:
		s.kind = ST_OUTER;
		s.a = value_opnd(L, in.a[0]);
		s.b = value_opnd(L, in.a[1]);
		s.o = value_opnd(L, in.out);
		s.p0 = (int)m->val[in.a[0]].n;
		s.p1 = (int)m->val[in.a[1]].n;
		break;
	case TGM_TAKE: {
		const tgm_shape &sw = m->val[in.a[0]].sh;
		s.kind = ST_TAKE;
		s.a = value_opnd(L, in.a[0]);
		s.b = value_opnd(L, in.a[1]);
		s.o = value_opnd(L, in.out);
		s.p0 = m->val[in.a[1]].sh.dim[0];
		s.p1 = sw.dim[0];
		s.p2 = (int)(numel(sw) / sw.dim[0]);
		break;
	}
	case TGM_SCAN: {
		for (int k = 0; k < in.nc; k++) {
			Step c;
			c.kind = ST_COPY;
			c.o = value_opnd(L, in.c[k]);
			c.a = value_opnd(L, in.cinit[k]);
			c.n = (int)m->val[in.c[k]].n;
			S.push_back(c);
		}
		Step fused;
		if (match_sscan(L, in, fused)) {
			S.push_back(fused);
			return true;
		}
		Step sc;
		sc.kind = ST_SCAN;
		sc.T = in.T;
		sc.reverse = in.reverse;
		sc.stid = in.stid;
		size_t at = S.size();
		S.push_back(sc);
		for (int j = 0; j < in.nx; j++) {
			Step c;
			c.kind = ST_COPY;
			c.o = value_opnd(L, in.xt[j]);
			c.a = value_opnd(L, in.x[j]);
			c.n = (int)m->val[in.xt[j]].n;
			c.dyn_a = 1;
			S.push_back(c);
		}
		if (!layer_block(L, in.body)) return false;
		for (int y = 0; y < in.ny; y++) {
			Step c;
			c.kind = ST_COPY;
			c.o = value_opnd(L, in.ys[y]);
			c.a = value_opnd(L, in.y[y]);
			c.n = (int)m->val[in.y[y]].n;
			c.dyn_o = 1;
			S.push_back(c);
		}
		for (int k = 0; k < in.nc; k++) {
			Step c;
			c.kind = ST_COPY;
			c.o = value_opnd(L, in.c[k]);
			c.a = value_opnd(L, in.cnext[k]);
			c.n = (int)m->val[in.c[k]].n;
			S.push_back(c);
		}
		S[at].body_lo = (int)at + 1;
		S[at].body_hi = (int)S.size();
		return true;
	}
	default:
		seterr("op '%s' is not supported by the layer executor", tgm_op_name(in.op));
		return false;
	}
	S.push_back(s);
	return true;
}

void mark_loop_values(const tgm_block *b, std::vector<char> &lw)
{
	for (int i = 0; i < b->len; i++) {
		const tgm_ins &in = b->v[i];
		if (in.op == TGM_SCAN) {
			for (int k = 0; k < in.nc; k++) lw[in.c[k]] = 1;
			for (int j = 0; j < in.nx; j++) lw[in.xt[j]] = 1;
			for (int y = 0; y < in.ny; y++) lw[in.ys[y]] = 1;
		}
		if (in.op == TGM_THINK) lw[in.out] = 1;
		if (in.body) mark_loop_values(in.body, lw);
	}
}

// how many times value v is read anywhere in block b (nested bodies included)
int value_reads(const tgm_block *b, int v)
{
	int n = 0;
	auto cnt = [&](const int *p, int k) {
		for (int i = 0; p && i < k; i++) n += p[i] == v;
	};
	for (int i = 0; i < b->len; i++) {
		const tgm_ins &in = b->v[i];
		cnt(in.a, in.na);
		if (in.op == TGM_THINK) n += (in.init == v) + (in.yield == v) + (in.halt == v);
		if (in.op == TGM_SCAN) {
			cnt(in.c, in.nc), cnt(in.cinit, in.nc), cnt(in.cnext, in.nc);
			cnt(in.x, in.nx), cnt(in.xt, in.nx), cnt(in.y, in.ny), cnt(in.ys, in.ny);
		}
		if (in.body) n += value_reads(in.body, v);
	}
	return n;
}

// the elementwise unary instructions (every one can sit in a GEMM epilogue chain)
bool epi_unary(int op)
{
	switch (op) {
	case TGM_NEG: case TGM_TANH: case TGM_RELU: case TGM_SIGMOID: case TGM_EXP: case TGM_SQRT: case TGM_GELU:
	case TGM_SILU: case TGM_SOFTPLUS: case TGM_LOG: case TGM_SIN: case TGM_COS: case TGM_FLOOR: case TGM_STEP: return true;
	default: return false;
	}
}

bool elementwise(int op) { return epi_unary(op) || (op >= TGM_ADD && op <= TGM_MIN); }

bool same_shape(const tgm_shape &x, const tgm_shape &y)
{
	if (x.rank != y.rank) return false;
	for (int i = 0; i < x.rank; i++)
		if (x.dim[i] != y.dim[i]) return false;
	return true;
}

// The instructions right after quantized product i of the top level that its
// GEMM can apply in its epilogue: a chain in which each instruction reads
// the previous one's result (read nowhere else, not the output, not a loop
// value) and keeps its shape, with up to TGK_EPI_MAX unary or binary
// instructions (the other operand of the output's shape, one value, or one
// value per channel) and then optionally a softmax or rmsnorm over the
// channels (C1's tanh, a bias, a residual add, C5's add then rmsnorm,
// qmlp's bias then softmax). The GEMM then writes the chain's last value,
// and the values are those of the instructions run apart, since the epilogue
// computes each with the elementwise kernels' arithmetic. Returns the index
// of the chain's last instruction (i: none).
int epi_chain(LB &L, const tgm_block *b, int i, Step &st)
{
	const tgm_module *m = L.m;
	const tgm_ins &in = b->v[i];
	const int quant = matmul_quant(m, in);
	const tgm_value &w = m->val[quant == 1 ? in.a[0] : in.a[1]];
	const tgm_shape &osh = m->val[in.out].sh;
	const int C = w.sh.dim[w.qaxis];
	// channel stride 1: x @ W ([.., C]) or W @ x for a vector x ([C])
	const bool chlast = osh.rank >= 1 && osh.dim[osh.rank - 1] == C && (quant == 2 || osh.rank == 1);
	auto single = [&](int v) { return v != m->output && !L.loopw[(size_t)v] && value_reads(&m->top, v) == 1; };
	int cur = in.out, j = i + 1;
	st.nepi = 0;
	st.rowop = 0;
	// a product whose activations another quantized product of the block also
	// reads keeps no chain: the GEMMs merge into one (merge_qgemms), which is
	// worth more (config 3's q/k/v and gate/up projections)
	const int act = quant == 1 ? in.a[1] : in.a[0];
	for (int k = 0; k < b->len; k++)
		if (k != i && b->v[k].op == TGM_MATMUL && matmul_quant(m, b->v[k])) {
			const int q2 = matmul_quant(m, b->v[k]);
			if ((q2 == 1 ? b->v[k].a[1] : b->v[k].a[0]) == act) return i;
		}
	while (j < b->len && single(cur)) {
		const tgm_ins &nx = b->v[j];
		if (st.nepi < TGK_EPI_MAX && epi_unary(nx.op) && nx.a[0] == cur) {
			st.epi[st.nepi++] = Step::Epi{ TGK_EW_UN, nx.op, 0, Opnd{} };
		} else if (st.nepi < TGK_EPI_MAX && nx.op >= TGM_ADD && nx.op <= TGM_MIN && (nx.a[0] == cur) != (nx.a[1] == cur) &&
			   same_shape(m->val[nx.out].sh, osh)) {
			const int other = nx.a[0] == cur ? nx.a[1] : nx.a[0];
			const tgm_shape &xs = m->val[other].sh;
			int mode = -1;
			if (same_shape(xs, osh)) mode = 0;
			else if (numel(xs) == 1) mode = 1;
			else if (chlast && numel(xs) == C && xs.rank >= 1 && xs.dim[xs.rank - 1] == C) mode = 3;
			if (mode < 0) break;
			st.epi[st.nepi++] = Step::Epi{ nx.a[0] == cur ? TGK_EW_BIN : TGK_EW_BINR, nx.op - TGM_ADD, mode, value_opnd(L, other) };
		} else if ((nx.op == TGM_RMSNORM || nx.op == TGM_SOFTMAX) && nx.a[0] == cur && chlast) {
			st.rowop = nx.op;
			st.p1 = C;
			st.p0 = (int)(numel(osh) / C);
			cur = nx.out;
			j++;
			break;
		} else
			break;
		cur = nx.out;
		j++;
	}
	// Worth it only if it saves memory traffic: when the next instruction is
	// elementwise and reads the chain's value, which nothing else reads, the
	// two would have been one fused elementwise run reading the product,
	// and the run now reads the chain's value instead (same bytes, a slower
	// GEMM epilogue). A row op, or a value read again later, saves a pass.
	if (!st.rowop && j < b->len && elementwise(b->v[j].op) && value_reads(&m->top, cur) == 1) {
		const tgm_ins &nx = b->v[j];
		bool reads = false;
		for (int k = 0; k < nx.na; k++) reads |= nx.a[k] == cur;
		if (reads) {
			st.nepi = 0;
			return i;
		}
	}
	return j - 1;
}

// A quantized product of the top block over many rows (16384 or more per
// pass) whose only reader is a lone tanh or silu takes that activation into
// its stores (qgemm_k's inline activation), where the chain rule would not
// give it one: the activation is not the next instruction, or the product
// shares its activations with another product and would merge with it
// (merge_qgemms; Mamba's in-projections x and z, whose x feeds a silu). Over
// that many rows the pass over the product it saves is worth more than the
// launch a merge saves. The activation is skipped by layer_block; its values
// are the elementwise kernel's (tg_ewop.h).
void plan_lone_acts(LB &L)
{
	const tgm_module *m = L.m;
	const tgm_block &b = m->top;
	if (L.p->flags & TG_HIP_EXACT) return;
	std::vector<int> uses((size_t)m->nval, 0), reader((size_t)m->nval, -1);
	count_uses(&b, uses);
	uses[(size_t)m->output]++;
	for (int i = 0; i < b.len; i++) {
		const tgm_ins &in = b.v[i];
		for (int j = 0; j < in.na; j++) reader[(size_t)in.a[j]] = i;
		if (in.op == TGM_SCAN) {
			for (int k = 0; k < in.nx; k++) reader[(size_t)in.x[k]] = i;
			for (int k = 0; k < in.nc; k++) reader[(size_t)in.cinit[k]] = i;
		}
	}
	auto act_of = [&](const tgm_ins &in) { return matmul_quant(m, in) == 1 ? in.a[1] : in.a[0]; };
	for (int i = 0; i < b.len; i++) {
		const tgm_ins &in = b.v[i];
		if (in.op != TGM_MATMUL || !matmul_quant(m, in) || L.skip[(size_t)i]) continue;
		const int v = in.out, k = reader[(size_t)v];
		if (uses[(size_t)v] != 1 || k <= i || L.loopw[(size_t)v] || L.skip[(size_t)k]) continue;
		const tgm_ins &nx = b.v[k];
		if ((nx.op != TGM_TANH && nx.op != TGM_SILU) || nx.na != 1 || nx.a[0] != v) continue;
		bool shared = false;
		for (int q = 0; q < b.len; q++)
			if (q != i && b.v[q].op == TGM_MATMUL && matmul_quant(m, b.v[q]) && act_of(b.v[q]) == act_of(in)) shared = true;
		if (!shared && k == i + 1) continue; // epi_chain takes it
		const tgm_value &w = m->val[matmul_quant(m, in) == 1 ? in.a[0] : in.a[1]];
		const long K = w.sh.rank == 2 ? w.sh.dim[1 - w.qaxis] : 0;
		if (K <= 0 || (long)L.p->max_rows * (numel(m->val[act_of(in)].sh) / K) < 16384) continue;
		L.lone[i] = k;
		L.skip[(size_t)k] = 1;
	}
}

bool layer_block(LB &L, const tgm_block *b)
{
	const bool top = b == &L.m->top;
	for (int i = 0; i < b->len; i++) {
		const tgm_ins &in = b->v[i];
		if (top && L.skip[(size_t)i]) continue; // folded into a fused scan (plan_sscan) or a product's stores (plan_lone_acts)
		if (top && L.lone.count(i)) { // the product applies its lone activation as it stores
			const tgm_ins &act = b->v[L.lone[i]];
			tgm_ins fused = in;
			fused.out = act.out;
			if (!layer_ins(L, fused)) return false;
			Step &st = L.p->steps.back();
			st.nepi = 1;
			st.epi[0] = Step::Epi{ TGK_EW_UN, act.op, 0, Opnd{} };
			L.p->stats.epilogue_ins += 1;
			continue;
		}
		if (in.op == TGM_MATMUL && top && !(L.p->flags & TG_HIP_EXACT) && matmul_quant(L.m, in)) {
			Step chain;
			int last = epi_chain(L, b, i, chain);
			for (int k = i + 1; k <= last; k++)
				if (L.skip[(size_t)k]) last = i; // (a chain never takes an instruction a scan folds in)
			if (last > i) { // the GEMM writes the chain's last value
				tgm_ins fused = in;
				fused.out = b->v[last].out;
				if (!layer_ins(L, fused)) return false;
				Step &st = L.p->steps.back();
				st.nepi = chain.nepi;
				for (int e = 0; e < chain.nepi; e++) st.epi[e] = chain.epi[e];
				st.rowop = chain.rowop;
				st.p0 = chain.p0;
				st.p1 = chain.p1;
				L.p->stats.epilogue_ins += chain.nepi + (chain.rowop != 0);
				i = last;
				continue;
			}
		}
		if (!layer_ins(L, in)) return false;
	}
	return true;
}

// -------------------------------------------------------- row program ----

struct RB {
	tg_hip_prog *p;
	tgm_module *m;
	Pools P;
	std::vector<int> ref; // value -> rp reference (INT_MIN: not yet placed)
	long slots = 0;
	bool fixed;
	long mult = 1; // executions per row of the instruction being built (think budgets and scan lengths)
};

int rp_ref(RB &B, int v)
{
	if (B.ref[v] != INT_MIN) return B.ref[v];
	const tgm_value &x = B.m->val[v];
	if (x.kind == TGM_PARAM || x.kind == TGM_STATE) {
		B.ref[v] = (int)(-pool_param(B.P, B.m, v, B.fixed) - 1);
	} else if (x.kind == TGM_INPUT) {
		B.ref[v] = B.p->rp_in_slot + (int)x.in_off;
	} else {
		B.ref[v] = (int)B.slots;
		B.slots += x.n;
	}
	return B.ref[v];
}

rp_ins rpi(int kind)
{
	rp_ins r;
	memset(&r, 0, sizeof r);
	r.kind = kind;
	return r;
}

int fbits(float f)
{
	int i;
	memcpy(&i, &f, 4);
	return i;
}

bool rp_block(RB &B, const tgm_block *b);

bool rp_ins_of(RB &B, const tgm_ins &in)
{
	tgm_module *m = B.m;
	auto &Pr = B.p->rprog;
	rp_ins r = rpi(RP_NOP);
	switch (in.op) {
	case TGM_CONST: {
		long off = (long)B.P.f.size();
		B.P.f.push_back(B.fixed ? fixed_word(in.k) : in.k);
		while (B.P.f.size() % 16) B.P.f.push_back(0.0f);
		B.ref[in.out] = (int)(-off - 1);
		return true;
	}
	case TGM_RESHAPE:
		r.kind = RP_COPY;
		r.out = rp_ref(B, in.out);
		r.a = rp_ref(B, in.a[0]);
		r.n = (int)m->val[in.out].n;
		break;
	case TGM_ADD: case TGM_SUB: case TGM_MUL: case TGM_DIV: case TGM_MAX: case TGM_MIN: {
		r.kind = RP_BIN;
		r.op = in.op - TGM_ADD;
		r.a = rp_ref(B, in.a[0]);
		r.b = rp_ref(B, in.a[1]);
		r.out = rp_ref(B, in.out);
		r.n = (int)m->val[in.out].n;
		long ao, bo;
		bcast(m->val[in.out].sh, m->val[in.a[0]].sh, B.P.imap, r.p[0], ao);
		bcast(m->val[in.out].sh, m->val[in.a[1]].sh, B.P.imap, r.p[2], bo);
		r.p[1] = (int)ao;
		r.p[3] = (int)bo;
		break;
	}
	case TGM_NEG: case TGM_TANH: case TGM_RELU: case TGM_SIGMOID: case TGM_EXP: case TGM_SQRT: case TGM_GELU:
	case TGM_SILU: case TGM_SOFTPLUS: case TGM_LOG: case TGM_SIN: case TGM_COS: case TGM_FLOOR: case TGM_STEP:
		r.kind = RP_UN;
		r.op = in.op;
		r.a = rp_ref(B, in.a[0]);
		r.out = rp_ref(B, in.out);
		r.n = (int)m->val[in.out].n;
		break;
	case TGM_MATMUL: {
		const tgm_value &va = m->val[in.a[0]], &vb = m->val[in.a[1]];
		int mm, kk, nn, gg;
		matmul_dims(va.sh, vb.sh, mm, kk, nn, gg);
		int quant = 0;
		if (gg == 1 && va.qbits && q_axis_for(m, in.a[0], in) == va.qaxis) quant = 1;
		else if (gg == 1 && vb.qbits && q_axis_for(m, in.a[1], in) == vb.qaxis) quant = 2;
		r.kind = RP_MM;
		r.out = rp_ref(B, in.out);
		r.a = quant == 1 ? 0 : rp_ref(B, in.a[0]);
		r.b = quant == 2 ? 0 : rp_ref(B, in.a[1]);
		r.p[0] = gg, r.p[1] = mm, r.p[2] = kk, r.p[3] = nn, r.p[4] = quant;
		if (!B.p->cap_of.empty() && gg == 1) { /* calibration samples, as src/quant.c:92-117 takes them */
			const int c0 = B.p->cap_of[in.a[0]], c1 = B.p->cap_of[in.a[1]];
			const bool left = c0 >= 0 && B.p->cap_axis[c0] == 0, right = c1 >= 0 && B.p->cap_axis[c1] == 1;
			if (left && right) B.p->cap_both = 1;
			const int c = left ? c0 : right ? c1 : -1;
			if (c >= 0) {
				r.p[8] = c + 1;
				r.p[9] = left ? 0 : 1;
				B.p->cap_rows[c] += (int)(B.mult * (left ? nn : mm));
			}
		}
		if (quant) {
			int v = quant == 1 ? in.a[0] : in.a[1];
			r.p[5] = m->val[v].qbits;
			r.p[6] = (int)pool_codes(B.P, m, v);
			r.p[7] = (int)B.P.scale_of[v];
		}
		break;
	}
	case TGM_SOFTMAX: case TGM_RMSNORM: {
		const tgm_shape &sa = m->val[in.a[0]].sh;
		r.kind = RP_ROW;
		r.op = in.op;
		r.a = rp_ref(B, in.a[0]);
		r.out = rp_ref(B, in.out);
		r.p[1] = sa.rank ? sa.dim[sa.rank - 1] : 1;
		r.p[0] = (int)(numel(sa) / r.p[1]);
		break;
	}
	case TGM_SUM: case TGM_MEAN:
		r.kind = RP_RED;
		r.op = in.op;
		r.a = rp_ref(B, in.a[0]);
		r.out = rp_ref(B, in.out);
		r.n = (int)m->val[in.a[0]].n;
		break;
	case TGM_TRANSPOSE: {
		const tgm_shape &sa = m->val[in.a[0]].sh;
		r.kind = RP_TRANS;
		r.a = rp_ref(B, in.a[0]);
		r.out = rp_ref(B, in.out);
		r.p[0] = sa.rank == 3 ? sa.dim[0] : 1;
		r.p[1] = sa.dim[sa.rank - 2];
		r.p[2] = sa.dim[sa.rank - 1];
		break;
	}
	case TGM_OUTER:
		r.kind = RP_OUTER;
		r.a = rp_ref(B, in.a[0]);
		r.b = rp_ref(B, in.a[1]);
		r.out = rp_ref(B, in.out);
		r.p[0] = (int)m->val[in.a[0]].n;
		r.p[1] = (int)m->val[in.a[1]].n;
		break;
	case TGM_TAKE: {
		const tgm_shape &sw = m->val[in.a[0]].sh;
		r.kind = RP_TAKE;
		r.a = rp_ref(B, in.a[0]);
		r.b = rp_ref(B, in.a[1]);
		r.out = rp_ref(B, in.out);
		r.p[0] = m->val[in.a[1]].sh.dim[0];
		r.p[1] = sw.dim[0];
		r.p[2] = (int)(numel(sw) / sw.dim[0]);
		break;
	}
	case TGM_THINK: {
		rp_ins t = rpi(RP_THINK);
		t.out = rp_ref(B, in.out);
		t.a = rp_ref(B, in.init);
		t.n = (int)m->val[in.out].n;
		t.p[1] = in.maxit;
		t.p[2] = in.eps >= 0 ? fbits(in.eps) : fbits(-1.0f);
		t.p[4] = fbits(in.hthr);
		t.p[5] = in.tid;
		if (in.eps >= 0) { // a positive threshold stays positive in Q16.16 (src/cgen.c:286-290)
			int32_t q = to_fixed(in.eps, 16);
			t.p[7] = (q > 0 || in.eps == 0) ? q : 1;
		}
		t.p[8] = to_fixed(in.hthr, 16);
		int at = (int)Pr.size();
		Pr.push_back(t);
		const long mult = B.mult;
		B.mult *= in.maxit;
		if (!rp_block(B, in.body)) return false;
		B.mult = mult;
		Pr[at].p[0] = rp_ref(B, in.yield);
		Pr[at].p[3] = in.halt >= 0 ? rp_ref(B, in.halt) : INT_MIN;
		rp_ins e = rpi(RP_THINK_END);
		e.p[0] = at;
		Pr.push_back(e);
		return true;
	}
	case TGM_SCAN: {
		for (int k = 0; k < in.nc; k++) {
			rp_ins c = rpi(RP_COPY);
			c.out = rp_ref(B, in.c[k]);
			c.a = rp_ref(B, in.cinit[k]);
			c.n = (int)m->val[in.c[k]].n;
			Pr.push_back(c);
		}
		rp_ins s = rpi(RP_SCAN);
		s.p[0] = in.T;
		s.p[1] = in.reverse;
		s.p[2] = in.stid;
		int at = (int)Pr.size();
		Pr.push_back(s);
		for (int j = 0; j < in.nx; j++) {
			rp_ins c = rpi(RP_COPY);
			c.out = rp_ref(B, in.xt[j]);
			c.a = rp_ref(B, in.x[j]);
			c.n = (int)m->val[in.xt[j]].n;
			c.p[2] = 1;
			Pr.push_back(c);
		}
		const long mult = B.mult;
		B.mult *= in.T;
		if (!rp_block(B, in.body)) return false;
		B.mult = mult;
		for (int y = 0; y < in.ny; y++) {
			rp_ins c = rpi(RP_COPY);
			c.out = rp_ref(B, in.ys[y]);
			c.a = rp_ref(B, in.y[y]);
			c.n = (int)m->val[in.y[y]].n;
			c.p[3] = 1;
			Pr.push_back(c);
		}
		for (int k = 0; k < in.nc; k++) {
			rp_ins c = rpi(RP_COPY);
			c.out = rp_ref(B, in.c[k]);
			c.a = rp_ref(B, in.cnext[k]);
			c.n = (int)m->val[in.c[k]].n;
			Pr.push_back(c);
		}
		rp_ins e = rpi(RP_SCAN_END);
		e.p[0] = at;
		Pr.push_back(e);
		return true;
	}
	default:
		seterr("op '%s' is not supported by the row executor", tgm_op_name(in.op));
		return false;
	}
	Pr.push_back(r);
	return true;
}

bool rp_block(RB &B, const tgm_block *b)
{
	for (int i = 0; i < b->len; i++)
		if (!rp_ins_of(B, b->v[i])) return false;
	return true;
}

template <class T>
bool upload(T **d, const std::vector<T> &h, hipStream_t st)
{
	size_t nb = (h.size() ? h.size() : 1) * sizeof(T);
	if (!hipok(hipMalloc((void **)d, nb), "hipMalloc")) return false;
	if (h.size() && !hipok(hipMemcpyAsync(*d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice, st), "upload")) return false;
	return true;
}

bool upload_pools(tg_hip_prog *p, Pools &P)
{
	return upload(&p->d_pool, P.f, p->st) && upload(&p->d_imap, P.imap, p->st) && upload(&p->d_codes, P.codes, p->st) &&
	       upload(&p->d_fscale, P.fscale, p->st) && upload(&p->d_qscale, P.qscale, p->st) &&
	       hipok(hipStreamSynchronize(p->st), "upload");
}

// ------------------------------------------------------------ execution ----

struct Run {
	tg_hip_prog *p;
	const float *in;
	float *out;
	int rows;
	int t; // current scan step
};

tgk_opd resolve(const Run &R, const Opnd &o)
{
	switch (o.space) {
	case SP_ARENA: return tgk_opd{ R.p->d_arena + o.off * (long)R.p->max_rows, o.rs };
	case SP_IN: return tgk_opd{ R.in + o.off, o.rs };
	case SP_POOL: return tgk_opd{ R.p->d_pool + o.off, 0 };
	case SP_OUT: return tgk_opd{ R.out, o.rs }; // the model's output is computed in place
	}
	return tgk_opd{ nullptr, 0 };
}

float *dst(const Run &R, const Opnd &o) { return const_cast<float *>(resolve(R, o).p); }

// With TG_HIP_TIMING every launch is bracketed by HIP events on the program's
// stream; `which` says where its time is accounted (0 other, 1 MFMA, 2 digits).
struct Timer {
	tg_hip_prog *p;
	hipEvent_t a = nullptr;
	int which;
	Timer(tg_hip_prog *p_, int w) : p(p_), which(w)
	{
		if (p->flags & TG_HIP_TIMING) {
			(void)hipEventCreate(&a);
			(void)hipEventRecord(a, p->st);
		}
	}
	~Timer()
	{
		if (!a) return;
		hipEvent_t b;
		(void)hipEventCreate(&b);
		(void)hipEventRecord(b, p->st);
		p->tev.push_back(a);
		p->tev.push_back(b);
		p->tev.push_back((hipEvent_t)(intptr_t)which);
	}
};

void exec_step(Run &R, const Step &s)
{
	tg_hip_prog *p = R.p;
	hipStream_t st = p->st;
	switch (s.kind) {
	case ST_BIN:
		tgk_binary(st, s.op, dst(R, s.o), s.o.rs, s.n, resolve(R, s.a), s.amode, p->d_imap + (s.amode == 2 ? s.amap : 0),
			   s.amode == 3 ? (int)s.amap : 1, resolve(R, s.b), s.bmode, p->d_imap + (s.bmode == 2 ? s.bmap : 0),
			   s.bmode == 3 ? (int)s.bmap : 1, R.rows);
		break;
	case ST_UN: tgk_unary(st, s.op, dst(R, s.o), s.o.rs, resolve(R, s.a), s.n, R.rows); break;
	case ST_MM: {
		tgk_mm d{};
		d.g = s.g, d.m = s.m, d.k = s.k, d.n = s.nn;
		d.a = s.quant == 1 ? tgk_opd{ nullptr, 0 } : resolve(R, s.a);
		d.ag = s.ag, d.ai = s.ai, d.ap = s.ap;
		d.b = s.quant == 2 ? tgk_opd{ nullptr, 0 } : resolve(R, s.b);
		d.bg = s.bg, d.bp = s.bp, d.bj = s.bj;
		d.o = dst(R, s.o);
		d.ors = s.o.rs, d.og = s.og, d.oi = s.oi, d.oj = s.oj;
		d.quant = s.quant, d.bits = s.bits;
		d.codes = p->d_codes + s.codes;
		d.scale = p->d_fscale + s.scale;
		tgk_matmul_exact(st, &d, R.rows);
		break;
	}
	case ST_NOP: break;
	case ST_QGEMM: {
		tgk_qgemm_args a;
		memset(&a, 0, sizeof a);
		a.w = &p->qws[s.qw];
		if (s.seg >= 0) {
			const std::vector<QSegOut> &g = p->qsegs[(size_t)s.seg];
			a.nseg = (int)g.size();
			for (size_t k = 0; k < g.size(); k++) {
				a.seg_c0[k] = g[k].c0;
				a.seg_o[k] = dst(R, g[k].o);
				a.seg_orr[k] = g[k].orr;
				a.seg_oj[k] = g[k].oj;
			}
			a.seg_c0[g.size()] = a.w->C;
		}
		tgk_opd x = resolve(R, s.a);
		a.x = x.p;
		a.xr = s.xr, a.xj = s.xj, a.xk = s.xk, a.ni = s.ni;
		a.o = dst(R, s.o);
		a.orr = s.orr, a.oc = s.oc, a.oj = s.ojj;
		a.M = R.rows * s.ni;
		a.nepi = s.nepi;
		for (int e = 0; e < s.nepi; e++) {
			const tgk_opd x = s.epi[e].kind == TGK_EW_UN ? tgk_opd{ nullptr, 0 } : resolve(R, s.epi[e].x);
			a.epi[e] = tgk_epi{ s.epi[e].kind, s.epi[e].op, s.epi[e].mode, x.p, x.rs };
		}
		a.rowop = s.rowop;
		int done;
		if (!s.reuse_digits && tgk_qgemm_fusable(&a)) { // one row: the digits are made inside the product's kernel
			Timer t(p, 1);
			done = tgk_qgemm_fused(st, &a, p->d_scratch);
		} else {
			if (!s.reuse_digits) {
				Timer t(p, 2);
				tgk_qgemm_digits(st, &a, p->d_scratch);
			}
			Timer t(p, 1);
			done = tgk_qgemm_mfma(st, &a, p->d_scratch);
		}
		if (s.nepi && !(done & TGK_DID_CHAIN)) { // a small-batch kernel: the chain over its output, in place
			Timer t(p, 3);
			tgk_qgemm_chain(st, &a);
		}
		if (s.rowop && !(done & TGK_DID_ROWOP)) { // no workgroup held whole lines: the row op over the output, in place
			Timer t(p, 3);
			tgk_rowop(st, s.rowop, a.o, s.o.rs, tgk_opd{ a.o, s.o.rs }, s.p0, s.p1, R.rows);
		}
		break;
	}
	case ST_ROW: tgk_rowop(st, s.op, dst(R, s.o), s.o.rs, resolve(R, s.a), s.p0, s.p1, R.rows); break;
	case ST_RED: tgk_reduce(st, s.op, dst(R, s.o), s.o.rs, resolve(R, s.a), s.n, R.rows); break;
	case ST_TRANS: tgk_transpose(st, dst(R, s.o), s.o.rs, resolve(R, s.a), s.p0, s.p1, s.p2, R.rows); break;
	case ST_OUTER: tgk_outer(st, dst(R, s.o), s.o.rs, resolve(R, s.a), s.p0, resolve(R, s.b), s.p1, R.rows); break;
	case ST_TAKE: tgk_take(st, dst(R, s.o), s.o.rs, resolve(R, s.a), resolve(R, s.b), s.p0, s.p1, s.p2, R.rows); break;
	case ST_COPY:
		tgk_copy(st, dst(R, s.o), s.o.rs, s.dyn_o ? (long)R.t * s.n : 0, resolve(R, s.a), s.dyn_a ? (long)R.t * s.n : 0, s.n,
			 R.rows);
		break;
	case ST_EW: {
		const EwStep &E = p->ews[(size_t)s.ew];
		tgk_ew e;
		memset(&e, 0, sizeof e);
		e.nin = (int)E.in.size();
		e.nout = (int)E.out.size();
		e.nins = (int)E.ins.size();
		for (int j = 0; j < e.nin; j++) {
			const tgk_opd x = resolve(R, E.in[(size_t)j].o);
			e.in[j] = x.p;
			e.in_rs[j] = x.rs;
			e.in_mode[j] = E.in[(size_t)j].mode;
			e.in_map[j] = E.in[(size_t)j].mode == 2 ? p->d_imap + E.in[(size_t)j].map : p->d_imap;
			e.in_per[j] = E.in[(size_t)j].mode == 3 ? (int)E.in[(size_t)j].map : 1;
			e.in_inv[j] = 1.0f / (float)e.in_per[j];
		}
		for (int j = 0; j < e.nout; j++) {
			e.out[j] = dst(R, E.out[(size_t)j]);
			e.out_rs[j] = E.out[(size_t)j].rs;
		}
		for (int k = 0; k < e.nins; k++) e.ins[k] = E.ins[(size_t)k];
		tgk_ew_run(st, &e, E.n, R.rows);
		break;
	}
	case ST_SSCAN: {
		tgk_sscan_fuse f{};
		if (s.fdu) f.dux = resolve(R, s.b);
		if (s.fgate) f.gx = resolve(R, s.f0), f.gD = resolve(R, s.f1).p, f.gz = resolve(R, s.f2);
		tgk_sscan(st, dst(R, s.o), s.o.rs, resolve(R, s.a), resolve(R, s.b), resolve(R, s.e0), resolve(R, s.e1), resolve(R, s.e2),
			  dst(R, s.e3), s.e3.rs, s.p0, s.p1, s.T, s.reverse, R.rows, &f);
		break;
	}
	}
}

void run_range(Run &R, int lo, int hi)
{
	tg_hip_prog *p = R.p;
	for (int i = lo; i < hi; i++) {
		const Step &s = p->steps[i];
		if (s.kind == ST_SCAN) {
			int saved = R.t;
			for (int step = 0; step < s.T; step++) {
				R.t = s.reverse ? s.T - 1 - step : step;
				run_range(R, s.body_lo, s.body_hi);
			}
			R.t = saved;
			i = s.body_hi - 1;
			continue;
		}
		if (s.kind == ST_QGEMM) {
			exec_step(R, s); /* times its two launches itself */
		} else {
			Timer t(p, 0);
			exec_step(R, s);
		}
	}
}

void collect_timing(tg_hip_prog *p)
{
	for (size_t i = 0; i + 3 <= p->tev.size(); i += 3) {
		float ms = 0;
		(void)hipEventElapsedTime(&ms, p->tev[i], p->tev[i + 1]);
		int which = (int)(intptr_t)p->tev[i + 2];
		if (which == 1) {
			p->stats.qgemm_ms += ms;
			p->stats.qgemm_calls++;
		} else if (which == 2) {
			p->stats.digits_ms += ms;
		} else {
			p->stats.other_ms += ms;
		}
		(void)hipEventDestroy(p->tev[i]);
		(void)hipEventDestroy(p->tev[i + 1]);
	}
	p->tev.clear();
}

// the steps of scans with a `steps` slot (fixed budget), row program excluded
void scan_tids(const tgm_block *b, std::vector<std::pair<int, int>> &out)
{
	for (int i = 0; i < b->len; i++) {
		if (b->v[i].op == TGM_SCAN && b->v[i].stid >= 0) out.push_back({ b->v[i].stid, b->v[i].T });
		if (b->v[i].body) scan_tids(b->v[i].body, out);
	}
}

int run_pass(tg_hip_prog *p, const float *d_in, int rows, float *d_out, int *d_steps)
{
	if (p->executor == 1 && p->rp_fn) {
		if (rows <= 0) return 0;
		const void *in = d_in;
		void *out = d_out;
		int *steps = d_steps;
		int r = rows;
		void *args[] = { &in, &out, &steps, &r };
		return hipok(hipModuleLaunchKernel(p->rp_fn, (unsigned)((rows + 255) / 256), 1, 1, 256, 1, 1, 0, p->st, args, nullptr),
			     "row program launch")
			       ? 0
			       : -1;
	}
	if (p->executor == 1) {
		rp_args a;
		memset(&a, 0, sizeof a);
		a.prog = p->d_rprog;
		a.nins = (int)p->rprog.size();
		a.pool = p->d_pool;
		a.imap = p->d_imap;
		a.codes = p->d_codes;
		a.fscale = p->d_fscale;
		a.qscale = p->d_qscale;
		a.arena = p->d_arena;
		a.arena_n = p->rp_arena;
		a.R = p->max_rows;
		a.in = d_in;
		a.per = (int)p->m->per;
		a.in_slot = p->rp_in_slot;
		a.out = d_out;
		a.nout = (int)p->m->nout;
		a.out_ref = p->rp_out_ref;
		a.steps = d_steps;
		a.nthink = p->m->nthink ? p->m->nthink : 1;
		a.rows = rows;
		a.fixed = p->fixed;
		a.cap = p->d_cap;
		a.cap_base = p->d_cap_base;
		a.cap_k = p->d_cap_k;
		a.cap_rows = p->d_cap_rows;
		a.cap_count = p->d_cap_count;
		tgk_rowprog(p->st, &a);
		return hipok(hipGetLastError(), "row program launch") ? 0 : -1;
	}
	Run R{ p, d_in, d_out, rows, 0 };
	run_range(R, 0, (int)p->steps.size());
	if (p->out.space != SP_OUT) {
		tgk_opd o = resolve(R, p->out);
		tgk_copy(p->st, d_out, p->m->nout, 0, o, 0, (int)p->m->nout, rows);
	}
	if (d_steps && p->m->nthink) {
		std::vector<std::pair<int, int>> t;
		scan_tids(&p->m->top, t);
		std::vector<int> h((size_t)rows * p->m->nthink, 0);
		for (int r = 0; r < rows; r++)
			for (auto &x : t) h[(size_t)r * p->m->nthink + x.first] = x.second;
		if (!hipok(hipMemcpyAsync(d_steps, h.data(), h.size() * sizeof(int), hipMemcpyHostToDevice, p->st), "steps")) return -1;
		if (!hipok(hipStreamSynchronize(p->st), "steps")) return -1;
	}
	return hipok(hipGetLastError(), "layer program launch") ? 0 : -1;
}

// ------------------------------------------------ quantized GEMMs ----

// activation digits depend on the activation operand, its strides and K
bool same_activation(const Step &x, const Step &y, const std::vector<tgk_qweight> &q)
{
	const tgk_qweight &a = q[(size_t)x.qw], &b = q[(size_t)y.qw];
	return same_value(x.a, y.a) && x.a.rs == y.a.rs && x.ni == y.ni && x.xr == y.xr && x.xj == y.xj && x.xk == y.xk && a.K == b.K &&
	       a.Kp == b.Kp;
}

// steps that a scan body runs (they may not move)
std::vector<char> in_scan(const std::vector<Step> &S)
{
	std::vector<char> in(S.size(), 0);
	for (size_t i = 0; i < S.size(); i++)
		if (S[i].kind == ST_SCAN)
			for (int j = S[i].body_lo; j < S[i].body_hi; j++) in[(size_t)j] = 1;
	return in;
}

// Quantized GEMMs of the top level that read the same activations (same
// operand, strides, K and weight width) become one GEMM over their weights
// concatenated along C, at the first one's place: its digits are computed
// once and narrow weights share tiles. Column c of member g is column
// c0[g] + c of the merged weight and goes to member g's output (TGK_QSEG
// output segments); every output value is the one the member computes alone.
// Moving a member up to the first one's place is safe: it reads only the
// activation, defined before the first one, and a param.
void merge_qgemms(tg_hip_prog *p, std::vector<std::vector<int8_t>> &mcodes, std::vector<std::vector<float>> &mscales)
{
	auto &S = p->steps;
	const std::vector<char> inscan = in_scan(S);
	std::vector<char> done(S.size(), 0);
	for (size_t i = 0; i < S.size(); i++) {
		if (S[i].kind != ST_QGEMM || inscan[i] || done[i] || S[i].nepi || S[i].rowop) continue;
		std::vector<size_t> g{ i };
		const tgk_qweight &w0 = p->qws[(size_t)S[i].qw];
		long ctot = w0.C;
		for (size_t j = i + 1; j < S.size() && g.size() < TGK_QSEG; j++) {
			const Step &t = S[j];
			if (t.kind != ST_QGEMM || inscan[j] || done[j] || t.nepi || t.rowop || !same_activation(S[i], t, p->qws) ||
			    t.oc != S[i].oc)
				continue;
			const tgk_qweight &w = p->qws[(size_t)t.qw];
			if (w.bits != w0.bits || ctot + w.C > (1L << 20)) continue;
			g.push_back(j);
			ctot += w.C;
		}
		if (g.size() < 2) continue;
		const tgm_module *m = p->m;
		const int K = w0.K;
		std::vector<int8_t> codes((size_t)ctot * K);
		std::vector<float> scales((size_t)ctot);
		std::vector<QSegOut> segs;
		long c0 = 0;
		for (size_t u : g) {
			const Step &t = S[u];
			const tgm_value &v = m->val[t.qv];
			const tgk_qweight &w = p->qws[(size_t)t.qw];
			for (int c = 0; c < w.C; c++) {
				for (int k = 0; k < K; k++)
					codes[(size_t)(c0 + c) * K + k] = (int8_t)tgm_code(&v, v.qaxis == 0 ? (long)c * K + k : (long)k * w.C + c);
				scales[(size_t)(c0 + c)] = v.qs[c];
			}
			segs.push_back({ t.o, (int)c0, t.orr, t.ojj });
			c0 += w.C;
			done[u] = 1;
		}
		tgk_qweight mw;
		memset(&mw, 0, sizeof mw);
		mw.C = (int)ctot, mw.K = K, mw.bits = w0.bits, mw.axis = 0;
		mw.Kp = w0.Kp, mw.Cp = (int)((ctot + 255) / 256 * 256);
		p->qws.push_back(mw);
		mcodes.resize(p->qws.size());
		mscales.resize(p->qws.size());
		mcodes.back() = std::move(codes);
		mscales.back() = std::move(scales);
		Step &h = S[i];
		h.qw = (int)p->qws.size() - 1;
		h.qv = -1;
		h.seg = (int)p->qsegs.size();
		p->qsegs.push_back(std::move(segs));
		for (size_t k = 1; k < g.size(); k++) S[g[k]].kind = ST_NOP;
	}
}

// Pack every weight a GEMM step uses: a merged weight from its concatenated
// codes, any other from its model value.
bool pack_weights(tg_hip_prog *p, std::vector<std::vector<int8_t>> &mcodes, std::vector<std::vector<float>> &mscales)
{
	mcodes.resize(p->qws.size());
	mscales.resize(p->qws.size());
	std::vector<char> used(p->qws.size(), 0);
	std::vector<int> src(p->qws.size(), -1);
	for (const Step &t : p->steps)
		if (t.kind == ST_QGEMM) used[(size_t)t.qw] = 1, src[(size_t)t.qw] = t.qv;
	for (size_t i = 0; i < p->qws.size(); i++) {
		tgk_qweight &w = p->qws[i];
		if (!used[i]) {
			memset(&w, 0, sizeof w);
			continue;
		}
		int rc;
		const char *name = "a merged weight";
		if (src[i] >= 0) {
			const tgm_value &v = p->m->val[src[i]];
			name = v.name ? v.name : "?";
			rc = tgk_qweight_pack(&w, v.q, v.qs, v.qbits, v.qaxis, w.C, w.K, p->st);
		} else {
			rc = tgk_qweight_pack_i8(&w, mcodes[i].data(), mscales[i].data(), w.bits, w.C, w.K, p->st);
		}
		std::vector<int8_t>().swap(mcodes[i]);
		std::vector<float>().swap(mscales[i]);
		if (rc) {
			seterr("cannot place the weights of %s on the device", name);
			return false;
		}
		p->stats.weight_bytes += (double)w.Cp * (w.bits == 8 ? w.Kp : w.Kp / 2) + 4.0 * w.Cp;
	}
	return true;
}

// A GEMM whose activation digits are already in the scratch: the last GEMM
// run before it, with nothing but non-GEMM steps between (which leave the
// scratch alone), read the same activations. Scan bodies start afresh.
void mark_digit_reuse(tg_hip_prog *p)
{
	auto &S = p->steps;
	const std::vector<char> inscan = in_scan(S);
	int last = -1;
	for (size_t i = 0; i < S.size(); i++) {
		Step &t = S[i];
		if (t.kind == ST_SCAN || (i > 0 && inscan[i] != inscan[i - 1])) last = -1;
		if (t.kind != ST_QGEMM) continue;
		t.reuse_digits = last >= 0 && !inscan[i] && same_activation(S[(size_t)last], t, p->qws);
		last = inscan[i] ? -1 : (int)i;
	}
}

// ------------------------------------------- rows read through take ----

void count_uses(const tgm_block *b, std::vector<int> &u)
{
	for (int i = 0; i < b->len; i++) {
		const tgm_ins &in = b->v[i];
		for (int j = 0; j < in.na; j++) u[(size_t)in.a[j]]++;
		if (in.op == TGM_SCAN) {
			for (int k = 0; k < in.nc; k++) u[(size_t)in.cinit[k]]++, u[(size_t)in.cnext[k]]++;
			for (int k = 0; k < in.nx; k++) u[(size_t)in.x[k]]++;
			for (int k = 0; k < in.ny; k++) u[(size_t)in.y[k]]++;
		}
		if (in.op == TGM_THINK) {
			u[(size_t)in.init]++;
			u[(size_t)in.yield]++;
			if (in.halt >= 0) u[(size_t)in.halt]++;
		}
		if (in.body) count_uses(in.body, u);
	}
}

// o = take(v, idx) with v = matmul(X, W) read by nothing else, X [M K] and W
// [K N] rank 2, idx a param whose entries all round into [0, M): row c of o
// is row idx[c] of X times W, so the program computes take(X, idx) and
// multiplies only those rows (the tied LM head of a decoder, read at the last
// position: one row instead of T). Each output row of a matmul depends only
// on its own input row, in every kernel here, so the values are unchanged.
// An index outside [0, M) would give a zero row, whose product with a W
// holding inf or nan is not zero: such indices keep the original program.
void push_take_into_matmul(tgm_module *m)
{
	tgm_block &b = m->top;
	std::vector<int> uses((size_t)m->nval, 0);
	count_uses(&b, uses);
	uses[(size_t)m->output]++;
	for (int i = 0; i < b.len; i++) {
		tgm_ins &tk = b.v[i];
		if (tk.op != TGM_TAKE || tk.na != 2) continue;
		const int v = tk.a[0], idx = tk.a[1];
		int j = i - 1;
		while (j >= 0 && b.v[j].out != v) j--;
		if (j < 0 || b.v[j].op != TGM_MATMUL || uses[(size_t)v] != 1) continue;
		tgm_ins &mm = b.v[j];
		const int X = mm.a[0], W = mm.a[1];
		const tgm_shape &sx = m->val[X].sh, &sw = m->val[W].sh;
		if (sx.rank != 2 || sw.rank != 2 || sx.dim[1] != sw.dim[0] || m->val[idx].kind != TGM_PARAM || !m->val[idx].data) continue;
		const int M = sx.dim[0], K = sx.dim[1];
		const long cnt = m->val[idx].n;
		bool in_range = cnt > 0;
		for (long c = 0; c < cnt && in_range; c++) {
			const float r = floorf(m->val[idx].data[c] + 0.5f);
			in_range = r >= 0.0f && r < (float)M;
		}
		if (!in_range) continue;
		if (m->nval == m->cap) {
			const int cap = m->cap ? 2 * m->cap : 64;
			tgm_value *nv = (tgm_value *)realloc(m->val, (size_t)cap * sizeof *nv);
			if (!nv) return; // keep the original program
			m->val = nv;
			m->cap = cap;
		}
		tgm_value &t = m->val[m->nval];
		memset(&t, 0, sizeof t);
		t.kind = TGM_TMP;
		t.sh.rank = 2;
		t.sh.dim[0] = (int)cnt;
		t.sh.dim[1] = K;
		t.n = cnt * K;
		const int tmp = m->nval++;
		mm.op = TGM_TAKE; // at the product's place (idx, a param, is defined throughout): tmp = take(X, idx)
		mm.out = tmp;
		mm.na = 2;
		mm.a[0] = X;
		mm.a[1] = idx;
		tk.op = TGM_MATMUL; // at the take's place: o = tmp @ W
		tk.a[0] = tmp;
		tk.a[1] = W;
	}
}

bool build_layer(tg_hip_prog *p)
{
	push_take_into_matmul(p->m);
	LB L;
	L.p = p;
	L.m = p->m;
	L.where.assign(p->m->nval, Opnd{});
	L.loopw.assign(p->m->nval, 0);
	L.P.pool_of.assign(p->m->nval, -1);
	L.P.codes_of.assign(p->m->nval, -1);
	L.P.scale_of.assign(p->m->nval, -1);
	mark_loop_values(&p->m->top, L.loopw);
	mark_transpose_views(L);
	plan_sscan(L);
	plan_lone_acts(L);
	if (p->m->val[p->m->output].kind == TGM_TMP) { /* written straight into the caller's output rows */
		L.where[p->m->output].space = SP_OUT;
		L.where[p->m->output].off = 0;
		L.where[p->m->output].rs = p->m->nout;
	}
	if (!layer_block(L, &p->m->top)) return false;
	p->out = value_opnd(L, p->m->output);
	std::vector<std::vector<int8_t>> mcodes;
	std::vector<std::vector<float>> mscales;
	merge_qgemms(p, mcodes, mscales);
	if (!pack_weights(p, mcodes, mscales)) return false;
	mark_digit_reuse(p);
	finish_ew(p);
	place_arena(p, p->m);
	if (!upload_pools(p, L.P)) return false;
	size_t ab = (size_t)(p->arena_floats ? p->arena_floats : 1) * p->max_rows * sizeof(float);
	p->stats.arena_bytes = (long)ab;
	if (!hipok(hipMalloc(&p->d_arena, ab), "arena")) return false;
	if (p->scratch_bytes && !hipok(hipMalloc(&p->d_scratch, p->scratch_bytes), "scratch")) return false;
	return true;
}

// the row program and its pools on the host
bool plan_rowprog(tg_hip_prog *p, RB &B)
{
	B.p = p;
	B.m = p->m;
	B.fixed = p->fixed != 0;
	B.ref.assign(p->m->nval, INT_MIN);
	B.P.pool_of.assign(p->m->nval, -1);
	B.P.codes_of.assign(p->m->nval, -1);
	B.P.scale_of.assign(p->m->nval, -1);
	p->rp_in_slot = 0;
	B.slots = p->m->per;
	if (!rp_block(B, &p->m->top)) return false;
	p->rp_out_ref = rp_ref(B, p->m->output);
	p->rp_arena = B.slots ? B.slots : 1;
	return true;
}

rp_source rp_source_of(const tg_hip_prog *p, const RB &B)
{
	rp_source r;
	r.prog = p->rprog.data();
	r.nins = (int)p->rprog.size();
	r.pool = B.P.f.data();
	r.npool = (long)B.P.f.size();
	r.imap = B.P.imap.data();
	r.codes = B.P.codes.data();
	r.fscale = B.P.fscale.data();
	r.qscale = B.P.qscale.data();
	r.per = (int)p->m->per;
	r.in_slot = p->rp_in_slot;
	r.nout = (int)p->m->nout;
	r.out_ref = p->rp_out_ref;
	r.nthink = p->m->nthink ? p->m->nthink : 1;
	r.arena = p->rp_arena;
	r.fixed = p->fixed != 0;
	return r;
}

// hipRTC compilation for the current device, cached per process by source text
bool rtc_compile(const std::string &src, std::vector<char> &code)
{
	static std::mutex mu;
	static std::map<std::string, std::vector<char>> cache;
	int dev = 0;
	hipDeviceProp_t pr;
	if (!hipok(hipGetDevice(&dev), "hipGetDevice") || !hipok(hipGetDeviceProperties(&pr, dev), "hipGetDeviceProperties")) return false;
	const std::string arch = std::string("--gpu-architecture=") + pr.gcnArchName;
	const std::string key = arch + "\n" + src;
	{
		std::lock_guard<std::mutex> g(mu);
		auto it = cache.find(key);
		if (it != cache.end()) {
			code = it->second;
			return true;
		}
	}
	hiprtcProgram prog;
	if (hiprtcCreateProgram(&prog, src.c_str(), "tg_rowprog.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS) {
		seterr("hiprtcCreateProgram failed");
		return false;
	}
	// the flags of the library's own kernels: no contraction, denormals kept, no packed FP32
	const char *opts[] = { arch.c_str(), "-O3", "-std=c++17", "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero",
		               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops" };
	hiprtcResult r = hiprtcCompileProgram(prog, (int)(sizeof opts / sizeof *opts), opts);
	if (r != HIPRTC_SUCCESS) {
		size_t n = 0;
		std::string log;
		if (hiprtcGetProgramLogSize(prog, &n) == HIPRTC_SUCCESS && n > 1) {
			log.resize(n);
			(void)hiprtcGetProgramLog(prog, &log[0]);
		}
		seterr("row program compilation failed: %.400s", log.c_str());
		(void)hiprtcDestroyProgram(&prog);
		return false;
	}
	size_t cs = 0;
	bool ok = hiprtcGetCodeSize(prog, &cs) == HIPRTC_SUCCESS && cs > 0;
	if (ok) {
		code.resize(cs);
		ok = hiprtcGetCode(prog, code.data()) == HIPRTC_SUCCESS;
	}
	(void)hiprtcDestroyProgram(&prog);
	if (!ok) {
		seterr("hiprtcGetCode failed");
		return false;
	}
	std::lock_guard<std::mutex> g(mu);
	cache[key] = code;
	return true;
}

// Compile the row program for this model. false with rp_why set: the program
// stays with the interpreter; false with an error: a failure to report.
bool compile_rowprog(tg_hip_prog *p, const RB &B, bool &fatal)
{
	fatal = false;
	std::string src;
	rp_emit_stats es;
	if (!rp_emit(rp_source_of(p, B), "tg_rowprog_model", false, src, p->rp_why, &es)) return false;
	std::vector<char> code;
	fatal = true;
	if (!rtc_compile(src, code)) return false;
	if (!hipok(hipModuleLoadData(&p->rp_mod, code.data()), "hipModuleLoadData")) return false;
	if (!hipok(hipModuleGetFunction(&p->rp_fn, p->rp_mod, "tg_rowprog_model"), "hipModuleGetFunction")) return false;
	p->stats.rowprog_jit = 1;
	p->stats.rowprog_hoisted = es.hoisted;
	fatal = false;
	return true;
}

bool build_rowprog(tg_hip_prog *p)
{
	RB B;
	if (!plan_rowprog(p, B)) return false;
	if (!(p->flags & TG_HIP_INTERP)) {
		bool fatal;
		if (compile_rowprog(p, B, fatal)) return true; // no arena, pools or program upload: all of it is in the kernel
		if (fatal) return false;
	} else {
		p->rp_why = "the interpreter was requested (TG_HIP_INTERP)";
	}
	if (!upload_pools(p, B.P) || !upload(&p->d_rprog, p->rprog, p->st)) return false;
	size_t ab = (size_t)p->rp_arena * p->max_rows * sizeof(float);
	p->stats.arena_bytes = (long)ab;
	return hipok(hipMalloc(&p->d_arena, ab), "arena") && hipok(hipStreamSynchronize(p->st), "upload");
}

void destroy(tg_hip_prog *p)
{
	if (!p) return;
	for (auto &q : p->qws) tgk_qweight_free(&q);
	void *bufs[] = { p->d_pool, p->d_imap, p->d_codes, p->d_fscale, p->d_qscale, p->d_arena, p->d_scratch, p->d_rprog, p->d_steps,
		         p->d_cap, p->d_cap_base, p->d_cap_k, p->d_cap_rows, p->d_cap_count };
	for (void *b : bufs)
		if (b) (void)hipFree(b);
	auto &h = p->hp;
	for (int k = 0; k < tg_hip_prog::NSL; k++) {
		void *dev[] = { h.d_in[k], h.d_out[k], h.d_steps[k] }, *host[] = { h.h_in[k], h.h_out[k], h.h_steps[k] };
		for (void *b : dev)
			if (b) (void)hipFree(b);
		for (void *b : host)
			if (b) (void)hipHostFree(b);
		hipEvent_t evs[] = { h.up[k], h.done[k], h.down[k], h.t0[k], h.t1[k] };
		for (hipEvent_t e : evs)
			if (e) (void)hipEventDestroy(e);
	}
	if (p->rp_mod) (void)hipModuleUnload(p->rp_mod);
	if (h.h2d) (void)hipStreamDestroy(h.h2d);
	if (h.d2h) (void)hipStreamDestroy(h.d2h);
	if (p->ev0) (void)hipEventDestroy(p->ev0);
	if (p->ev1) (void)hipEventDestroy(p->ev1);
	if (p->own_st) (void)hipStreamDestroy(p->own_st);
	tgm_free(p->m);
	delete p;
}

// memcpy on a few host threads (pageable caller memory <-> pinned staging)
void par_copy(void *dst, const void *src, size_t n)
{
	const size_t piece = (size_t)4 << 20;
	const int nt = n < 2 * piece ? 1 : (int)std::min<size_t>(8, n / piece);
	if (nt == 1) {
		memcpy(dst, src, n);
		return;
	}
	std::vector<std::thread> th;
	const size_t per = (n + nt - 1) / nt;
	for (int t = 0; t < nt; t++) {
		const size_t a = (size_t)t * per, b = std::min(n, a + per);
		if (a < b) th.emplace_back([=] { memcpy((char *)dst + a, (const char *)src + a, b - a); });
	}
	for (auto &x : th) x.join();
}

// Pinned host allocations made by tg_hip_host_alloc: start -> size. A row or
// output buffer inside one moves over PCIe directly (no staging copy).
std::mutex g_pinned_mu;
std::map<uintptr_t, size_t> g_pinned;

bool in_pinned(const void *h, size_t bytes)
{
	if (!h) return false;
	const uintptr_t a = (uintptr_t)h;
	std::lock_guard<std::mutex> lk(g_pinned_mu);
	auto it = g_pinned.upper_bound(a);
	if (it == g_pinned.begin()) return false;
	--it;
	return a - it->first <= it->second && bytes <= it->second - (a - it->first);
}

bool host_pipe_init(tg_hip_prog *p)
{
	auto &h = p->hp;
	if (h.chunk) return true;
	const long per = p->m->per, nout = p->m->nout, nt = p->m->nthink ? p->m->nthink : 1;
	// about 16 MiB of rows per chunk: copies of one chunk overlap the compute of the next
	long c = (16l << 20) / (4 * (per > nout ? per : nout));
	c = c < 256 ? 256 : c;
	h.chunk = c < p->max_rows ? c : p->max_rows;
	bool ok = hipok(hipStreamCreate(&h.h2d), "stream") && hipok(hipStreamCreate(&h.d2h), "stream");
	for (int k = 0; ok && k < tg_hip_prog::NSL; k++)
		ok = hipok(hipHostMalloc(&h.h_in[k], (size_t)h.chunk * per * 4, 0), "pinned input") &&
		     hipok(hipHostMalloc(&h.h_out[k], (size_t)h.chunk * nout * 4, 0), "pinned output") &&
		     hipok(hipHostMalloc((void **)&h.h_steps[k], (size_t)h.chunk * nt * 4, 0), "pinned steps") &&
		     hipok(hipMalloc(&h.d_in[k], (size_t)h.chunk * per * 4), "input buffer") &&
		     hipok(hipMalloc(&h.d_out[k], (size_t)h.chunk * nout * 4), "output buffer") &&
		     hipok(hipMalloc(&h.d_steps[k], (size_t)h.chunk * nt * 4), "steps buffer") &&
		     hipok(hipEventCreateWithFlags(&h.up[k], hipEventDisableTiming), "event") &&
		     hipok(hipEventCreateWithFlags(&h.done[k], hipEventDisableTiming), "event") &&
		     hipok(hipEventCreateWithFlags(&h.down[k], hipEventDisableTiming), "event") && hipok(hipEventCreate(&h.t0[k]), "event") &&
		     hipok(hipEventCreate(&h.t1[k]), "event");
	if (!ok) h.chunk = 0;
	return ok;
}

// Host buffers, the block loop of `tgc batch`: rows go in chunks through a
// three-slot pipeline. Chunk i uses slot i % 3: its rows are copied into the
// slot's pinned buffer on the host, up to the device on the copy-in stream,
// computed on the program's stream, and down on the copy-out stream; each
// stream waits for the event of the step before it, and a slot is refilled
// only after its previous chunk has left it. So chunk i + 1 travels while
// chunk i computes. Passes run in input order on one stream, as before.
// Rows, outputs or steps in memory from tg_hip_host_alloc skip the host
// copies: the transfers read and write the caller's buffers directly.
int batch_host(tg_hip_prog *p, const void *rows, long nrows, void *out, int *steps)
{
	if (!p) {
		seterr("no program");
		return -1;
	}
	if (!host_pipe_init(p)) return -1;
	auto &h = p->hp;
	const long per = p->m->per, nout = p->m->nout, nt = p->m->nthink ? p->m->nthink : 1;
	const bool din = in_pinned(rows, (size_t)nrows * per * 4), dout = in_pinned(out, (size_t)nrows * nout * 4);
	const bool dsteps = steps && in_pinned(steps, (size_t)nrows * nt * 4);
	// chunks of about 16 MiB of rows through the staging slots (the host copies
	// want large pieces); a quarter of that when nothing is staged, so the
	// first chunk's upload and the last one's download, which nothing
	// overlaps, are short
	const long C = din && dout ? std::max(64L, h.chunk / 4) : h.chunk;
	const long nch = (nrows + C - 1) / C;
	float ms_total = 0;
	auto finish = [&](long i) -> bool { // chunk i's outputs to the caller
		const int k = (int)(i % tg_hip_prog::NSL);
		const long r0 = i * C, cnt = nrows - r0 < C ? nrows - r0 : C;
		if (!hipok(hipEventSynchronize(h.down[k]), "outputs to host")) return false;
		if (!dout) par_copy((char *)out + (size_t)r0 * nout * 4, h.h_out[k], (size_t)cnt * nout * 4);
		if (steps && p->m->nthink && !dsteps) memcpy(steps + (size_t)r0 * nt, h.h_steps[k], (size_t)cnt * nt * 4);
		float ms = 0;
		(void)hipEventElapsedTime(&ms, h.t0[k], h.t1[k]);
		ms_total += ms;
		return true;
	};
	for (long i = 0; i < nch; i++) {
		const int k = (int)(i % tg_hip_prog::NSL);
		const long r0 = i * C, cnt = nrows - r0 < C ? nrows - r0 : C;
		if (i >= tg_hip_prog::NSL && !finish(i - tg_hip_prog::NSL)) return -1; // the slot's previous chunk is out: its buffers are free
		const void *src = (const char *)rows + (size_t)r0 * per * 4;
		if (!din) {
			par_copy(h.h_in[k], src, (size_t)cnt * per * 4);
			src = h.h_in[k];
		}
		if (!hipok(hipMemcpyAsync(h.d_in[k], src, (size_t)cnt * per * 4, hipMemcpyHostToDevice, h.h2d), "rows to device") ||
		    !hipok(hipEventRecord(h.up[k], h.h2d), "event") || !hipok(hipStreamWaitEvent(p->st, h.up[k], 0), "wait"))
			return -1;
		(void)hipEventRecord(h.t0[k], p->st);
		if (run_pass(p, h.d_in[k], (int)cnt, h.d_out[k], h.d_steps[k])) return -1;
		(void)hipEventRecord(h.t1[k], p->st);
		void *odst = dout ? (void *)((char *)out + (size_t)r0 * nout * 4) : h.h_out[k];
		void *sdst = dsteps ? (void *)(steps + (size_t)r0 * nt) : (void *)h.h_steps[k];
		if (!hipok(hipEventRecord(h.done[k], p->st), "event") || !hipok(hipStreamWaitEvent(h.d2h, h.done[k], 0), "wait") ||
		    !hipok(hipMemcpyAsync(odst, h.d_out[k], (size_t)cnt * nout * 4, hipMemcpyDeviceToHost, h.d2h), "outputs to host"))
			return -1;
		if (steps && p->m->nthink &&
		    !hipok(hipMemcpyAsync(sdst, h.d_steps[k], (size_t)cnt * nt * 4, hipMemcpyDeviceToHost, h.d2h), "steps to host"))
			return -1;
		if (!hipok(hipEventRecord(h.down[k], h.d2h), "event")) return -1;
	}
	for (long i = nch > tg_hip_prog::NSL ? nch - tg_hip_prog::NSL : 0; i < nch; i++)
		if (!finish(i)) return -1;
	collect_timing(p);
	if (steps && !p->m->nthink) memset(steps, 0, (size_t)nrows * sizeof *steps); /* no think loop: one zero slot per row */
	p->stats.rows = (int)nrows;
	p->stats.batch_ms = ms_total;
	return 0;
}

} // namespace

// for the decoder (tg_decode.cpp): the program's model and stream
const tgm_module *tgh_prog_module(const tg_hip_prog *p) { return p->m; }
hipStream_t tgh_prog_stream(const tg_hip_prog *p) { return p->st; }
void tgh_set_error(const char *msg) { seterr("%s", msg); }

extern "C" {

int tg_hip_init(int device)
{
	if (!hipok(hipSetDevice(device), "hipSetDevice")) return -1;
	return scratch_on(device) ? 0 : -1; // the no-allocation entry point's scratch on this device
}

// A device program; with `cap` (calibration), the row-program interpreter with
// the products of the listed params capturing their samples.
tg_hip_prog *load_prog(const char *tgir, size_t len, int flags, int max_rows, const tgq_param *cap, int ncap)
{
	char err[512];
	tgm_module *m = tgm_read(tgir, len, err, sizeof err);
	if (!m) {
		seterr("%s", err);
		return nullptr;
	}
	if (m->nupd) {
		seterr("model %s updates its state: rows depend on each other and stay on the CPU", m->name);
		tgm_free(m);
		return nullptr;
	}
	tg_hip_prog *p = new tg_hip_prog;
	p->m = m;
	if (cap) {
		flags |= TG_HIP_ROWPROG | TG_HIP_INTERP;
		p->cap_of.assign(m->nval, -1);
		for (int i = 0; i < ncap; i++) {
			p->cap_of[cap[i].v] = i;
			p->cap_axis.push_back(cap[i].axis);
		}
		p->cap_rows.assign(ncap, 0);
	}
	p->flags = flags;
	p->fixed = (flags & TG_HIP_FIXED) != 0;
	p->max_rows = max_rows > 0 ? max_rows : 4096;
	p->executor = (p->fixed || (flags & TG_HIP_ROWPROG) || has_think(&m->top)) ? 1 : 0;
	p->stats.executor = p->executor;
	bool ok = hipok(hipStreamCreate(&p->own_st), "hipStreamCreate") && hipok(hipEventCreate(&p->ev0), "event") &&
		  hipok(hipEventCreate(&p->ev1), "event");
	p->st = p->own_st;
	if (ok) ok = p->executor ? build_rowprog(p) : build_layer(p);
	if (!ok) {
		destroy(p);
		return nullptr;
	}
	return p;
}

tg_hip_prog *tg_hip_load(const char *tgir, size_t len, int flags, int max_rows)
{
	return load_prog(tgir, len, flags, max_rows, nullptr, 0);
}

const char *tg_hip_model_name(const tg_hip_prog *p) { return p ? p->m->name : ""; }

int tg_hip_signature(const tg_hip_prog *p, char *json, size_t n)
{
	if (!p || !json || !n) return -1;
	std::string s = std::string("{\"model\":\"") + p->m->name + "\",\"inputs\":[";
	auto type = [](const tgm_shape &sh) {
		std::string t = "(f32";
		for (int i = 0; i < sh.rank; i++) t += " " + std::to_string(sh.dim[i]);
		return t + ")";
	};
	for (int i = 0; i < p->m->ninputs; i++) {
		const tgm_value &v = p->m->val[p->m->inputs[i]];
		s += std::string(i ? "," : "") + "{\"name\":\"" + v.name + "\",\"type\":\"" + type(v.sh) + "\"}";
	}
	s += "],\"output\":\"" + type(p->m->val[p->m->output].sh) + "\",\"values_per_row\":" + std::to_string(p->m->per) +
	     ",\"think_loops\":" + std::to_string(p->m->nthink) + ",\"stateful\":" + (p->m->nupd ? "true" : "false") + "}\n";
	snprintf(json, n, "%s", s.c_str());
	return s.size() < n ? (int)s.size() : -1;
}

int tg_hip_info(const tg_hip_prog *p, int *per, int *nout, int *nthink)
{
	if (!p) return -1;
	if (per) *per = (int)p->m->per;
	if (nout) *nout = (int)p->m->nout;
	if (nthink) *nthink = p->m->nthink;
	return 0;
}

int tg_hip_batch(tg_hip_prog *p, const float *rows, long nrows, float *out, int *steps)
{
	if (p && p->fixed) {
		seterr("this program runs in Q16.16: use tg_hip_batch_fixed");
		return -1;
	}
	return batch_host(p, rows, nrows, out, steps);
}

int tg_hip_batch_fixed(tg_hip_prog *p, const int32_t *rows, long nrows, int32_t *out, int *steps)
{
	if (p && !p->fixed) {
		seterr("this program runs in f32: load it with TG_HIP_FIXED");
		return -1;
	}
	return batch_host(p, rows, nrows, out, steps);
}

int tg_hip_batch_device(tg_hip_prog *p, const void *d_rows, long nrows, void *d_out, int *d_steps)
{
	if (!p) return -1;
	if (nrows > p->max_rows) {
		seterr("%ld rows exceed the program's %d-row capacity", nrows, p->max_rows);
		return -1;
	}
	if (!d_steps && p->m->nthink) {
		if (!p->d_steps && !hipok(hipMalloc(&p->d_steps, (size_t)p->max_rows * p->m->nthink * 4), "steps buffer")) return -1;
		d_steps = p->d_steps;
	}
	if (!p->span_open) {
		(void)hipEventRecord(p->ev0, p->st);
		p->span_open = true;
	}
	int rc = run_pass(p, (const float *)d_rows, (int)nrows, (float *)d_out, d_steps);
	p->stats.rows = (int)nrows;
	return rc;
}

int tg_hip_sync(tg_hip_prog *p)
{
	if (!p) return -1;
	/* the span's end is marked here, not after every call: an event per call
	   would put a queue barrier between back-to-back batches */
	if (p->span_open && !hipok(hipEventRecord(p->ev1, p->st), "event")) return -1;
	if (!hipok(hipStreamSynchronize(p->st), "sync")) return -1;
	float ms = 0;
	if (p->span_open && hipEventElapsedTime(&ms, p->ev0, p->ev1) == hipSuccess) p->stats.batch_ms = ms;
	p->span_open = false;
	collect_timing(p);
	return 0;
}

int tg_hip_set_stream(tg_hip_prog *p, void *stream)
{
	if (!p) return -1;
	if (!hipok(hipStreamSynchronize(p->st), "set_stream")) return -1; /* finish what is queued on the old stream */
	p->st = stream ? (hipStream_t)stream : p->own_st;
	p->span_open = false;
	return 0;
}

void *tg_hip_get_stream(const tg_hip_prog *p) { return p ? (void *)p->st : nullptr; }

int tg_hip_matmul_qa(float *o, const signed char *q, int bits, const float *s, const float *b, int m, int k, int n)
{
	return tg_hip_matmul_q(o, q, bits, s, b, m, k, n, 0, 0);
}

int tg_hip_matmul_qb(float *o, const float *a, const signed char *q, int bits, const float *s, int m, int k, int n)
{
	return tg_hip_matmul_q(o, q, bits, s, a, m, k, n, 1, 0);
}

int tg_hip_matmul_q(float *o, const signed char *q, int bits, const float *s, const float *b, int m, int k, int n, int axis, int flags)
{
	if ((bits != 8 && bits != 4) || (axis != 0 && axis != 1) || m < 1 || k < 1 || n < 1) {
		seterr("tg_hip_matmul_q: bad arguments");
		return -1;
	}
	hipStream_t st;
	if (!hipok(hipStreamCreate(&st), "stream")) return -1;
	int rc = -1;
	long nq = (long)(axis == 0 ? m : k) * (axis == 0 ? k : n), qb = bits == 8 ? nq : (nq + 1) / 2;
	long bn = axis == 0 ? (long)k * n : (long)m * k, on = (long)m * n, nch = axis == 0 ? m : n;
	float *db = nullptr, *dout = nullptr, *ds = nullptr;
	uint8_t *dq = nullptr;
	void *scr = nullptr;
	tgk_qweight w{};
	do {
		if (!hipok(hipMalloc(&db, bn * 4), "alloc") || !hipok(hipMalloc(&dout, on * 4), "alloc")) break;
		if (!hipok(hipMemcpyAsync(db, b, bn * 4, hipMemcpyHostToDevice, st), "copy")) break;
		if (flags & TG_HIP_EXACT) {
			if (!hipok(hipMalloc(&dq, qb), "alloc") || !hipok(hipMalloc(&ds, nch * 4), "alloc")) break;
			(void)hipMemcpyAsync(dq, q, qb, hipMemcpyHostToDevice, st);
			(void)hipMemcpyAsync(ds, s, nch * 4, hipMemcpyHostToDevice, st);
			tgk_mm d{};
			d.g = 1, d.m = m, d.k = k, d.n = n;
			d.quant = axis == 0 ? 1 : 2;
			d.bits = bits;
			d.codes = dq;
			d.scale = ds;
			d.a = tgk_opd{ axis == 1 ? db : nullptr, 0 };
			d.ai = k, d.ap = 1;
			d.b = tgk_opd{ axis == 0 ? db : nullptr, 0 };
			d.bp = n, d.bj = 1;
			d.o = dout;
			d.oi = n, d.oj = 1;
			tgk_matmul_exact(st, &d, 1);
		} else {
			int C = axis == 0 ? m : n, K = k;
			if (tgk_qweight_pack(&w, (const uint8_t *)q, s, bits, axis, C, K, st)) {
				seterr("tg_hip_matmul_q: weight upload failed");
				break;
			}
			tgk_qgemm_args a{};
			a.w = &w;
			a.x = db;
			a.o = dout;
			if (axis == 0) { // rows j of b^T: element k at k * n
				a.ni = n, a.xr = 0, a.xj = 1, a.xk = n, a.M = n;
				a.orr = 0, a.oc = n, a.oj = 1;
			} else {
				a.ni = m, a.xr = 0, a.xj = k, a.xk = 1, a.M = m;
				a.orr = 0, a.oc = 1, a.oj = n;
			}
			if (!hipok(hipMalloc(&scr, tgk_qgemm_scratch(a.M, w.Kp)), "alloc")) break;
			tgk_qgemm(st, &a, scr);
		}
		if (!hipok(hipGetLastError(), "launch")) break;
		if (!hipok(hipMemcpyAsync(o, dout, on * 4, hipMemcpyDeviceToHost, st), "copy")) break;
		if (!hipok(hipStreamSynchronize(st), "sync")) break;
		rc = 0;
	} while (0);
	tgk_qweight_free(&w);
	void *bufs[] = { db, dout, ds, dq, scr };
	for (void *x : bufs)
		if (x) (void)hipFree(x);
	(void)hipStreamDestroy(st);
	return rc;
}

int tg_hip_matmul_q_noalloc(float *d_o, const signed char *d_q, int bits, const float *d_s, const float *d_b, int m, int k, int n,
			    int axis, void *stream)
{
	if ((bits != 8 && bits != 4) || (axis != 0 && axis != 1) || m < 1 || k < 1 || n < 1 || !d_o || !d_q || !d_s || !d_b) {
		seterr("tg_hip_matmul_q_noalloc: bad arguments");
		return -1;
	}
	const int C = axis == 0 ? m : n, K = k, M = axis == 0 ? n : m;
	const size_t wb = tgk_qweight_dev_bytes(bits, C, K), Kp = (size_t)(K + 63) / 64 * 64;
	const size_t need = wb + tgk_qgemm_scratch(M, (int)Kp);
	if (need > TG_HIP_NOALLOC_SCRATCH) {
		seterr("tg_hip_matmul_q_noalloc: %d x %d weights with %d activation rows need %zu bytes of scratch, more than "
		       "the %u the library holds (TG_HIP_NOALLOC_SCRATCH)", C, K, M, need, (unsigned)TG_HIP_NOALLOC_SCRATCH);
		return -2;
	}
	int dev = 0;
	if (!hipok(hipGetDevice(&dev), "hipGetDevice")) return -1;
	uint8_t *scr = (uint8_t *)scratch_on(dev);
	if (!scr) return -1;
	hipStream_t st = (hipStream_t)stream;
	tgk_qweight w;
	if (tgk_qweight_pack_dev(&w, scr, (const uint8_t *)d_q, d_s, bits, axis, C, K, st)) {
		seterr("tg_hip_matmul_q_noalloc: weight packing launch failed");
		return -1;
	}
	tgk_qgemm_args a{};
	a.w = &w;
	a.x = d_b;
	a.o = d_o;
	if (axis == 0) { // rows j of b^T: element k at k * n
		a.ni = n, a.xr = 0, a.xj = 1, a.xk = n, a.M = n;
		a.orr = 0, a.oc = n, a.oj = 1;
	} else {
		a.ni = m, a.xr = 0, a.xj = k, a.xk = 1, a.M = m;
		a.orr = 0, a.oc = 1, a.oj = n;
	}
	tgk_qgemm(st, &a, scr + wb); // digits, then the matrix-core product (every byte they read is written first)
	return hipok(hipGetLastError(), "tg_hip_matmul_q_noalloc launch") ? 0 : -1;
}

char *tg_hip_emit_unit(const char *tgir, size_t len, int flags, const char *kernel)
{
	char err[512];
	tgm_module *m = tgm_read(tgir, len, err, sizeof err);
	if (!m) {
		seterr("%s", err);
		return nullptr;
	}
	if (m->nupd) {
		seterr("model %s updates its state: rows depend on each other", m->name);
		tgm_free(m);
		return nullptr;
	}
	std::string name = kernel ? kernel : "";
	if (name.empty()) {
		name = "tg_";
		for (const char *c = m->name; c && *c; c++) name += (isalnum((unsigned char)*c) || *c == '_') ? *c : '_';
		name += "_rows";
	}
	tg_hip_prog *p = new tg_hip_prog;
	p->m = m;
	p->flags = flags;
	p->fixed = (flags & TG_HIP_FIXED) != 0;
	p->max_rows = 1;
	RB B;
	std::string src;
	char *out = nullptr;
	if (plan_rowprog(p, B)) {
		if (rp_emit(rp_source_of(p, B), name.c_str(), true, src, p->rp_why, nullptr)) {
			out = (char *)malloc(src.size() + 1);
			if (out) memcpy(out, src.c_str(), src.size() + 1);
			else seterr("out of memory");
		} else {
			seterr("model %s: %s", m->name, p->rp_why.c_str());
		}
	}
	destroy(p);
	return out;
}

void tg_hip_str_free(char *s) { free(s); }

char *tg_hip_surface_to_tgir(const char *path)
{
	char err[1024];
	char *t = path ? tgf_lower(path, err, sizeof err) : nullptr;
	if (!t) seterr("%s", path ? err : "no model path");
	return t;
}

namespace {

// The f32 model over the calibration rows in one device pass of the row
// interpreter, capturing every listed param's samples; each param's Hessian
// summed on the device in the reference's order (tgk_hessian) and copied to
// q[i].H (malloc'd) with its sample count. The outputs go to ref.
int calibrate(const char *tgir, size_t len, tgq_param *q, int n, const float *calib, long ncalib, std::vector<float> &ref)
{
	if (ncalib > INT_MAX) {
		seterr("too many calibration rows");
		return -1;
	}
	tg_hip_prog *p = load_prog(tgir, len, 0, (int)ncalib, q, n);
	if (!p) return -1;
	auto fail = [&](void *a, void *b, void *c, void *d) {
		for (void *x : { a, b, c, d })
			if (x) (void)hipFree(x);
		destroy(p);
		return -1;
	};
	if (p->cap_both) {
		seterr("a product of two eligible params: its calibration samples are not captured");
		return fail(nullptr, nullptr, nullptr, nullptr);
	}
	const long per = p->m->per, nout = p->m->nout, nt = p->m->nthink ? p->m->nthink : 1;
	std::vector<long> base(n);
	std::vector<int> ks(n);
	long tot = 0;
	for (int i = 0; i < n; i++)
		if (q[i].K > 65535) {
			seterr("a layer %d inputs wide gets no Hessian on this backend (at most 65535)", q[i].K);
			return fail(nullptr, nullptr, nullptr, nullptr);
		}
	for (int i = 0; i < n; i++) {
		base[i] = tot;
		ks[i] = q[i].K;
		tot += ncalib * (long)p->cap_rows[i] * q[i].K;
	}
	if (tot > (8L << 30) / 4) {
		seterr("calibration samples need %ld MiB of device memory", tot * 4 >> 20);
		return fail(nullptr, nullptr, nullptr, nullptr);
	}
	float *d_in = nullptr, *d_out = nullptr;
	int *d_steps = nullptr;
	double *d_h = nullptr;
	bool ok = hipok(hipMalloc(&p->d_cap, (size_t)(tot ? tot : 1) * 4), "calibration samples") &&
		  upload(&p->d_cap_base, base, p->st) && upload(&p->d_cap_k, ks, p->st) && upload(&p->d_cap_rows, p->cap_rows, p->st) &&
		  hipok(hipMalloc(&p->d_cap_count, (size_t)n * ncalib * sizeof(int) + 4), "calibration counts") &&
		  hipok(hipMemsetAsync(p->d_cap_count, 0, (size_t)n * ncalib * sizeof(int) + 4, p->st), "memset") &&
		  hipok(hipMalloc(&d_in, (size_t)ncalib * per * 4), "calibration rows") &&
		  hipok(hipMalloc(&d_out, (size_t)ncalib * nout * 4), "calibration outputs") &&
		  hipok(hipMalloc(&d_steps, (size_t)ncalib * nt * 4), "calibration steps") &&
		  hipok(hipMemcpyAsync(d_in, calib, (size_t)ncalib * per * 4, hipMemcpyHostToDevice, p->st), "upload");
	if (!ok || tg_hip_batch_device(p, d_in, ncalib, d_out, d_steps) || tg_hip_sync(p)) return fail(d_in, d_out, d_steps, nullptr);
	ref.resize((size_t)ncalib * nout);
	std::vector<int> cnt((size_t)n * ncalib);
	ok = hipok(hipMemcpy(ref.data(), d_out, ref.size() * 4, hipMemcpyDeviceToHost), "download") &&
	     hipok(hipMemcpy(cnt.data(), p->d_cap_count, cnt.size() * 4, hipMemcpyDeviceToHost), "download");
	for (size_t i = 0; ok && i < cnt.size(); i++)
		if (cnt[i] > p->cap_rows[i / ncalib]) {
			seterr("internal: %d calibration samples of param %d in a row, room for %d", cnt[i], (int)(i / ncalib), p->cap_rows[i / ncalib]);
			ok = false;
		}
	for (int i = 0; ok && i < n; i++) {
		if (!p->cap_rows[i]) continue; /* never in a product the hook sees */
		const size_t kk = (size_t)q[i].K * q[i].K;
		q[i].H = (double *)malloc(kk * sizeof(double));
		ok = q[i].H && hipok(hipMalloc(&d_h, kk * sizeof(double)), "Hessian");
		if (!ok) break;
		tgk_hessian(p->st, p->d_cap + base[i], p->d_cap_count + (long)i * ncalib, p->cap_rows[i], q[i].K, (int)ncalib, d_h);
		ok = hipok(hipGetLastError(), "Hessian launch") && hipok(hipMemcpyAsync(q[i].H, d_h, kk * sizeof(double), hipMemcpyDeviceToHost, p->st), "download") &&
		     hipok(hipStreamSynchronize(p->st), "Hessian");
		(void)hipFree(d_h);
		d_h = nullptr;
		q[i].nsamp = 0;
		for (long r = 0; r < ncalib; r++) q[i].nsamp += cnt[(size_t)i * ncalib + r];
	}
	if (!ok) return fail(d_in, d_out, d_steps, d_h);
	fail(d_in, d_out, d_steps, nullptr);
	return 0;
}

// the model's outputs over rows on the device (default path)
int run_outputs(const char *tgir, size_t len, const float *rows, long n, std::vector<float> &out)
{
	tg_hip_prog *p = tg_hip_load(tgir, len, 0, n > 4096 ? 4096 : (int)n);
	if (!p) return -1;
	out.resize((size_t)n * p->m->nout);
	std::vector<int> steps((size_t)n * (p->m->nthink ? p->m->nthink : 1));
	int rc = tg_hip_batch(p, rows, n, out.data(), steps.data());
	destroy(p);
	return rc;
}

} // namespace

char *tg_hip_quantize_model(const char *tgir, size_t len, int bits, int gptq, const float *calib, long ncalib, int min_size, int max_k,
			    long *bytes, char *log, size_t logn)
{
	char dummy[1];
	if (!log || !logn) log = dummy, logn = 1;
	log[0] = 0;
	if (bits != 8 && bits != 4) {
		seterr("bits is 8 or 4");
		return nullptr;
	}
	if (gptq && (!calib || ncalib < 1)) {
		seterr("GPTQ needs calibration rows (input rows in the tgc batch format)");
		return nullptr;
	}
	char err[512];
	tgm_module *m = tgm_read(tgir, len, err, sizeof err);
	if (!m) {
		seterr("%s", err);
		return nullptr;
	}
	tgq_param *q = nullptr;
	int n = m->nupd ? 0 : tgq_eligible(m, min_size, &q);
	char *out = nullptr;
	std::vector<float> ref, got;
	if (m->nupd) {
		seterr("model %s updates its state: it stays on the CPU path", m->name);
	} else if (n <= 0) {
		seterr("%s: no param is eligible (rank-2, >= %d elements, used only as a matmul operand)", m->name, min_size);
	} else {
		bool ok = true;
		if (gptq) { /* Hessians for every param (max_k <= 0), or as the reference for K <= max_k */
			std::vector<tgq_param> cap;
			std::vector<int> idx;
			for (int i = 0; i < n; i++)
				if (max_k <= 0 || q[i].K <= max_k) cap.push_back(q[i]), idx.push_back(i);
			ok = cap.empty() || calibrate(tgir, len, cap.data(), (int)cap.size(), calib, ncalib, ref) == 0;
			for (size_t j = 0; j < idx.size(); j++) q[idx[j]].H = cap[j].H, q[idx[j]].nsamp = cap[j].nsamp;
		} else if (calib && ncalib > 0) {
			ok = run_outputs(tgir, len, calib, ncalib, ref) == 0;
		}
		if (ok) {
			snprintf(log, logn, "quantize: %d param(s) of %s\n", n, m->name);
			const int threads = (int)std::max(1u, std::min(64u, std::thread::hardware_concurrency()));
			for (int i = 0; ok && i < n; i++) ok = tgq_quantize_param(m, &q[i], bits, gptq, threads, log, logn) == 0;
			if (!ok) seterr("out of memory quantizing");
		}
		if (ok && !(out = tgm_write(m))) seterr("out of memory writing the model");
		if (out && bytes) { /* the params' bytes before and after (src/quant.c:352-360) */
			bytes[0] = bytes[1] = 0;
			for (int v = 0; v < m->nval; v++) {
				const tgm_value *x = &m->val[v];
				if (x->kind != TGM_PARAM) continue;
				bytes[0] += 4 * x->n;
				bytes[1] += x->qbits ? (x->qbits == 8 ? x->n : (x->n + 1) / 2) + 4L * x->sh.dim[x->qaxis] : 4 * x->n;
			}
		}
		if (out && !ref.empty() && run_outputs(out, strlen(out), calib, ncalib, got) == 0 && got.size() == ref.size()) {
			double num = 0, den = 0, mx = 0; /* what quantization does to the outputs on the calibration rows */
			for (size_t i = 0; i < ref.size(); i++) {
				double d = (double)got[i] - ref[i];
				num += d * d;
				den += (double)ref[i] * ref[i];
				mx = std::max(mx, std::fabs(d));
			}
			size_t o = strlen(log);
			snprintf(log + o, logn - o, "quantize: on %ld calibration row(s): relative output error %.5f, max |output change| %.5f\n", ncalib,
				 den > 0 ? std::sqrt(num / den) : 0.0, mx);
		}
	}
	for (int i = 0; i < n; i++) free(q[i].H);
	free(q);
	tgm_free(m);
	return out;
}

void tg_hip_free(tg_hip_prog *p) { destroy(p); }

const char *tg_hip_error(void) { return g_err; }

int tg_hip_stats(const tg_hip_prog *p, tg_hip_stats_t *st)
{
	if (!p || !st) return -1;
	*st = p->stats;
	return 0;
}

int tg_hip_reset_stats(tg_hip_prog *p)
{
	if (!p) return -1;
	p->stats.qgemm_ms = p->stats.other_ms = p->stats.digits_ms = 0;
	p->stats.qgemm_calls = 0;
	return 0;
}

int tg_hip_read_pass(const void *d, size_t bytes, int blocks, void *stream)
{
	static int *sink = nullptr; // one int per process, never read
	if (!d || ((size_t)d & 15) || blocks <= 0) {
		seterr("tg_hip_read_pass: bad arguments");
		return -1;
	}
	if (!sink && !hipok(hipMalloc(&sink, sizeof(int)), "hipMalloc")) return -1;
	tgk_read((hipStream_t)stream, d, bytes, blocks, sink);
	return hipok(hipGetLastError(), "read pass launch") ? 0 : -1;
}

void *tg_hip_dev_alloc(size_t bytes)
{
	void *d = nullptr;
	if (!hipok(hipMalloc(&d, bytes ? bytes : 1), "hipMalloc")) return nullptr;
	return d;
}

int tg_hip_dev_free(void *d) { return hipok(hipFree(d), "hipFree") ? 0 : -1; }

void *tg_hip_host_alloc(size_t bytes)
{
	void *h = nullptr;
	if (!hipok(hipHostMalloc(&h, bytes ? bytes : 1, 0), "pinned host memory")) return nullptr;
	std::lock_guard<std::mutex> lk(g_pinned_mu);
	g_pinned[(uintptr_t)h] = bytes;
	return h;
}

int tg_hip_host_free(void *h)
{
	if (!h) return 0;
	{
		std::lock_guard<std::mutex> lk(g_pinned_mu);
		auto it = g_pinned.find((uintptr_t)h);
		if (it == g_pinned.end()) {
			seterr("tg_hip_host_free: not a tg_hip_host_alloc pointer");
			return -1;
		}
		g_pinned.erase(it);
	}
	return hipok(hipHostFree(h), "hipHostFree") ? 0 : -1;
}
int tg_hip_h2d(void *d, const void *h, size_t bytes) { return hipok(hipMemcpy(d, h, bytes, hipMemcpyHostToDevice), "h2d") ? 0 : -1; }
int tg_hip_d2h(void *h, const void *d, size_t bytes) { return hipok(hipMemcpy(h, d, bytes, hipMemcpyDeviceToHost), "d2h") ? 0 : -1; }

} // extern "C"
