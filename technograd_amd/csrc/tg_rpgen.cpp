// Row programs compiled for one model (tg_rpgen.h). The emitted kernel runs
// one batch row per lane, like the interpreter, but with the program unrolled
// into straight-line code: arena slots become variables (so values stay in
// registers instead of the [slot][lane] device arena), and operands that the
// interpreter reads from the pools become literals.
//
// Think loops (src/vm.c:383-411, src/cgen.c:265-311) become real loops with
// the same exit tests in the same order. An instruction of a think body is
// hoisted in front of the loop when every slot it reads is written neither in
// the body nor by the loop's state update (or only by instructions hoisted
// before it): it then computes the same value at every iteration, and a think
// body runs at least once, so computing it once is exact. In the latent
// reasoner this moves `w_inj @ e` (a 16 x 16 product) out of the loop.
#include "tg_rpgen.h"
#include "tgm.h"

#include <climits>
#include <cstdio>
#include <cstring>
#include <utility>
#include <vector>

namespace {

// the element functions, as text (generated from tg_devmath.h and tg_rowdev.h at build time)
const char DEVMATH_TEXT[] =
#include "tg_devmath.inc"
	;
const char ROWDEV_TEXT[] =
#include "tg_rowdev.inc"
	;

constexpr long MAX_SLOTS = 1024;     // variables per lane (beyond this they would live in scratch memory)
constexpr long MAX_TERMS = 1L << 14; // multiply-add terms (compile time grows with the text)

struct Node {
	int ins = -1;           // instruction index; an RP_THINK heads a loop
	std::vector<Node> body; // the loop's body
	std::vector<Node> pre;  // instructions hoisted in front of the loop
};

std::string itos(long v) { return std::to_string(v); }

bool parse(const rp_source &S, int &pc, int think, std::vector<Node> &out, std::string &why)
{
	while (pc < S.nins) {
		const rp_ins &I = S.prog[pc];
		switch (I.kind) {
		case RP_THINK_END:
			if (I.p[0] != think) {
				why = "unbalanced think loop";
				return false;
			}
			return true;
		case RP_SCAN: case RP_SCAN_STEP: case RP_SCAN_END:
			why = "scan loops run in the interpreter";
			return false;
		case RP_TAKE:
			why = "take (a data-dependent gather) runs in the interpreter";
			return false;
		case RP_COPY:
			if (I.p[2] || I.p[3]) {
				why = "scan slices run in the interpreter";
				return false;
			}
			break;
		case RP_UN:
			if (I.op < TGM_NEG || I.op > TGM_STEP) {
				why = "unknown element function";
				return false;
			}
			break;
		case RP_BIN: case RP_MM: case RP_ROW: case RP_RED: case RP_TRANS: case RP_OUTER: case RP_THINK: case RP_NOP:
			break;
		default:
			why = "instruction kind not compiled";
			return false;
		}
		Node n;
		n.ins = pc;
		if (I.kind == RP_THINK) {
			int at = pc++;
			if (!parse(S, pc, at, n.body, why)) return false;
			if (pc >= S.nins) {
				why = "unterminated think loop";
				return false;
			}
		}
		if (I.kind != RP_NOP) out.push_back(std::move(n));
		pc++;
	}
	if (think >= 0) why = "unterminated think loop";
	return think < 0;
}

// element index of a broadcast operand (mode 0: same index, 1: element 0, 2: index map)
long bidx(const rp_source &S, int mode, int off, long i) { return mode == 0 ? i : mode == 1 ? 0 : S.imap[off + i]; }

// slots an instruction reads and writes (pool operands are not slots)
void access(const rp_source &S, const rp_ins &I, std::vector<long> &rd, std::vector<long> &wr)
{
	auto R = [&](int ref, long i) {
		if (ref >= 0) rd.push_back(ref + i);
	};
	auto W = [&](int ref, long i) {
		if (ref >= 0) wr.push_back(ref + i);
	};
	switch (I.kind) {
	case RP_BIN:
		for (long i = 0; i < I.n; i++) {
			R(I.a, bidx(S, I.p[0], I.p[1], i));
			R(I.b, bidx(S, I.p[2], I.p[3], i));
			W(I.out, i);
		}
		break;
	case RP_UN:
		for (long i = 0; i < I.n; i++) R(I.a, i), W(I.out, i);
		break;
	case RP_MM: {
		const long G = I.p[0], M = I.p[1], K = I.p[2], N = I.p[3];
		if (I.p[4] != 1)
			for (long e = 0; e < G * M * K; e++) R(I.a, e);
		if (I.p[4] != 2)
			for (long e = 0; e < G * K * N; e++) R(I.b, e);
		for (long e = 0; e < G * M * N; e++) W(I.out, e);
		break;
	}
	case RP_ROW:
		for (long e = 0; e < (long)I.p[0] * I.p[1]; e++) R(I.a, e), W(I.out, e);
		break;
	case RP_RED:
		for (long i = 0; i < I.n; i++) R(I.a, i);
		W(I.out, 0);
		break;
	case RP_TRANS:
		for (long e = 0; e < (long)I.p[0] * I.p[1] * I.p[2]; e++) R(I.a, e), W(I.out, e);
		break;
	case RP_OUTER:
		for (long i = 0; i < I.p[0]; i++) R(I.a, i);
		for (long j = 0; j < I.p[1]; j++) R(I.b, j);
		for (long e = 0; e < (long)I.p[0] * I.p[1]; e++) W(I.out, e);
		break;
	case RP_COPY:
		for (long i = 0; i < I.n; i++) R(I.a, I.p[1] + i), W(I.out, I.p[0] + i);
		break;
	default: break;
	}
}

void node_writes(const rp_source &S, const Node &n, std::vector<long> &wr)
{
	const rp_ins &I = S.prog[n.ins];
	if (I.kind != RP_THINK) {
		std::vector<long> rd;
		access(S, I, rd, wr);
		return;
	}
	for (long i = 0; i < I.n; i++) wr.push_back(I.out + i); // initial copy and the per-iteration state update
	for (auto &c : n.pre) node_writes(S, c, wr);
	for (auto &c : n.body) node_writes(S, c, wr);
}

void hoist(const rp_source &S, Node &loop, long &count)
{
	// inner loops first: what leaves an inner loop joins this body in front of it
	std::vector<Node> nb;
	for (auto &c : loop.body) {
		if (S.prog[c.ins].kind == RP_THINK) {
			hoist(S, c, count);
			for (auto &h : c.pre) nb.push_back(std::move(h));
			c.pre.clear();
		}
		nb.push_back(std::move(c));
	}
	loop.body.swap(nb);
	std::vector<int> wc(S.arena, 0); // writes of each slot within one iteration (state update included)
	std::vector<long> wr;
	for (long i = 0; i < S.prog[loop.ins].n; i++) wr.push_back(S.prog[loop.ins].out + i);
	for (auto &c : loop.body) node_writes(S, c, wr);
	for (long s : wr) wc[s]++;
	std::vector<char> hw(S.arena, 0); // written by a hoisted instruction
	std::vector<Node> keep;
	for (auto &c : loop.body) {
		bool ok = S.prog[c.ins].kind != RP_THINK;
		std::vector<long> rd, w;
		if (ok) {
			access(S, S.prog[c.ins], rd, w);
			for (long s : rd)
				if (wc[s] && !hw[s]) ok = false;
			for (long s : w)
				if (wc[s] != 1) ok = false;
		}
		if (ok) {
			for (long s : w) hw[s] = 1;
			loop.pre.push_back(std::move(c));
			count++;
		} else {
			keep.push_back(std::move(c));
		}
	}
	loop.body.swap(keep);
}

struct Gen {
	const rp_source &S;
	bool fx;
	std::string out;
	int depth = 1;
	std::vector<char> used;
	long terms = 0;
	int loops = 0;

	explicit Gen(const rp_source &s) : S(s), fx(s.fixed), used(s.arena, 0) {}

	void ln(const std::string &t)
	{
		out.append((size_t)depth, '\t');
		out += t;
		out += '\n';
	}
	std::string slot(long s)
	{
		used[s] = 1;
		return "v" + itos(s);
	}
	static std::string ilit(long v) { return v == INT_MIN ? std::string("(-2147483647 - 1)") : itos(v); }
	static std::string flit(float f)
	{
		unsigned u;
		memcpy(&u, &f, 4);
		char b[40];
		snprintf(b, sizeof b, "__int_as_float(0x%08x)", u);
		return b;
	}
	std::string word(long w)
	{
		float f = S.pool[w];
		if (!fx) return flit(f);
		int q;
		memcpy(&q, &f, 4);
		return ilit(q);
	}
	std::string rd(int ref, long i) { return ref >= 0 ? slot(ref + i) : word(-(long)ref - 1 + i); }
	std::string wr(int ref, long i) { return slot(ref + i); }
	int code(long off, int bits, long i) const
	{
		const uint8_t *q = S.codes + off;
		if (bits == 8) return (signed char)q[i];
		int b = (signed char)q[i >> 1];
		return (i & 1) ? (b >> 4) : (int)(signed char)(unsigned char)((unsigned)b << 4) >> 4;
	}

	std::string bin(int op, const std::string &x, const std::string &y)
	{
		if (fx) {
			static const char *f[] = { "addq", "subq", "fmulq", "fdivq", "maxq", "minq" };
			return std::string("tgrd::") + f[op] + "(" + x + ", " + y + ")";
		}
		switch (op) {
		case TGK_ADD: return x + " + " + y;
		case TGK_SUB: return x + " - " + y;
		case TGK_MUL: return x + " * " + y;
		case TGK_DIV: return x + " / " + y;
		case TGK_MAX: return "tgrd::maxf_(" + x + ", " + y + ")";
		default: return "tgrd::minf_(" + x + ", " + y + ")";
		}
	}
	std::string un(int op, const std::string &x)
	{
		static const char *q[] = { "tgrd::negq", "tgrd::tanhq", "tgrd::reluq", "tgrd::sigmoidq", "tgrd::expq",
			                   "tgrd::sqrtq", "tgrd::geluq", "tgrd::siluq", "tgrd::softplusq", "tgrd::logq",
			                   "tgrd::sinq", "tgrd::cosq", "tgrd::floorq", "tgrd::stepq" };
		static const char *f[] = { "tgrd::negf_", "tanhf", "tgrd::reluf_", "tgrd::sigmoidf_", "expf", "sqrtf",
			                   "tgrd::geluf_", "tgrd::siluf_", "tgrd::softplusf_", "logf", "sinf", "cosf", "floorf",
			                   "tgrd::stepf_" };
		return std::string(fx ? q[op - TGM_NEG] : f[op - TGM_NEG]) + "(" + x + ")";
	}

	bool mm(const rp_ins &I)
	{
		const long G = I.p[0], M = I.p[1], K = I.p[2], N = I.p[3];
		const int quant = I.p[4], bits = I.p[5];
		if ((terms += G * M * N * K) > MAX_TERMS) return false;
		for (long g = 0; g < G; g++)
			for (long i = 0; i < M; i++)
				for (long j = 0; j < N; j++) {
					const long ai = g * M * K + i * K, bj = g * K * N + j, oi = g * M * N + i * N + j;
					std::string t = fx ? "{ long s = 0;" : "{ float s = 0.0f;";
					for (long p = 0; p < K; p++) {
						std::string x, y;
						if (quant == 1) {
							int c = code(I.p[6], bits, i * K + p);
							if (fx && c == 0) continue; // adds 0 to an integer sum
							x = fx ? itos(c) : itos(c) + ".0f";
							y = rd(I.b, bj + p * N);
						} else if (quant == 2) {
							int c = code(I.p[6], bits, p * N + j);
							if (fx && c == 0) continue;
							x = rd(I.a, ai + p);
							y = fx ? itos(c) : itos(c) + ".0f";
						} else {
							x = rd(I.a, ai + p);
							y = rd(I.b, bj + p * N);
						}
						t += fx ? " s += (long)" + x + " * " + y + ";" : " s = s + " + x + " * " + y + ";";
						if (p % 8 == 7 && p + 1 < K) {
							ln(t);
							t = "  ";
						}
					}
					if (quant) {
						const long c = I.p[7] + (quant == 1 ? i : j);
						t += " " + wr(I.out, oi) + (fx ? " = tgrd::qscaleq(s, " + ilit(S.qscale[c]) + ");" : " = " + flit(S.fscale[c]) + " * s;");
					} else {
						t += " " + wr(I.out, oi) + (fx ? " = tgrd::sat((s + 32768) >> 16);" : " = s;");
					}
					ln(t + " }");
				}
		return true;
	}

	void row(const rp_ins &I)
	{
		const long nrow = I.p[0], cols = I.p[1];
		for (long q = 0; q < nrow; q++) {
			const long b = q * cols;
			ln("{");
			depth++;
			if (I.op == TGM_SOFTMAX) {
				ln(std::string(fx ? "int" : "float") + " mx = " + rd(I.a, b) + ";");
				for (long i = 1; i < cols; i++)
					ln(fx ? "mx = " + rd(I.a, b + i) + " > mx ? " + rd(I.a, b + i) + " : mx;" : "if (" + rd(I.a, b + i) + " > mx) mx = " + rd(I.a, b + i) + ";");
				ln(fx ? "long s = 0;" : "float s = 0.0f;");
				for (long i = 0; i < cols; i++) {
					if (fx) ln(wr(I.out, b + i) + " = tgrd::expq_neg(tgrd::subq(" + rd(I.a, b + i) + ", mx)); s += " + rd(I.out, b + i) + ";");
					else ln(wr(I.out, b + i) + " = expf(" + rd(I.a, b + i) + " - mx); s = s + " + rd(I.out, b + i) + ";");
				}
				for (long i = 0; i < cols; i++)
					ln(wr(I.out, b + i) + (fx ? " = tgrd::softq(" + rd(I.out, b + i) + ", s);" : " = " + rd(I.out, b + i) + " / s;"));
			} else { // rmsnorm
				ln(fx ? "unsigned long ss = 0;" : "float s = 0.0f;");
				for (long i = 0; i < cols; i++) {
					const std::string x = rd(I.a, b + i);
					ln(fx ? "ss += (unsigned long)((long)" + x + " * " + x + ");" : "s = s + " + x + " * " + x + ";");
				}
				ln(fx ? "const int rms = tgrd::rmsq(ss, " + itos(cols) + ");" : "const float inv = 1.0f / sqrtf(s / " + itos(cols) + ".0f + 1e-6f);");
				for (long i = 0; i < cols; i++)
					ln(wr(I.out, b + i) + (fx ? " = tgrd::fdivq(" + rd(I.a, b + i) + ", rms);" : " = " + rd(I.a, b + i) + " * inv;"));
			}
			depth--;
			ln("}");
		}
	}

	bool ins(const rp_ins &I)
	{
		switch (I.kind) {
		case RP_BIN:
			for (long i = 0; i < I.n; i++)
				ln(wr(I.out, i) + " = " + bin(I.op, rd(I.a, bidx(S, I.p[0], I.p[1], i)), rd(I.b, bidx(S, I.p[2], I.p[3], i))) + ";");
			break;
		case RP_UN:
			for (long i = 0; i < I.n; i++) ln(wr(I.out, i) + " = " + un(I.op, rd(I.a, i)) + ";");
			break;
		case RP_MM:
			return mm(I);
		case RP_ROW:
			row(I);
			break;
		case RP_RED: {
			std::string t = fx ? "{ long s = 0;" : "{ float s = 0.0f;";
			for (long i = 0; i < I.n; i++) t += fx ? " s += " + rd(I.a, i) + ";" : " s = s + " + rd(I.a, i) + ";";
			if (I.op == TGM_SUM) t += " " + wr(I.out, 0) + (fx ? " = tgrd::sat(s); }" : " = s; }");
			else t += " " + wr(I.out, 0) + (fx ? " = tgrd::sat(s / " + itos(I.n) + "); }" : " = s / " + itos(I.n) + ".0f; }");
			ln(t);
			break;
		}
		case RP_TRANS: {
			const long G = I.p[0], RR = I.p[1], C = I.p[2];
			for (long z = 0; z < G; z++)
				for (long i = 0; i < RR; i++)
					for (long j = 0; j < C; j++) ln(wr(I.out, z * RR * C + j * RR + i) + " = " + rd(I.a, z * RR * C + i * C + j) + ";");
			break;
		}
		case RP_OUTER:
			for (long i = 0; i < I.p[0]; i++)
				for (long j = 0; j < I.p[1]; j++)
					ln(wr(I.out, i * I.p[1] + j) + " = " + (fx ? "tgrd::fmulq(" + rd(I.a, i) + ", " + rd(I.b, j) + ")" : rd(I.a, i) + " * " + rd(I.b, j)) + ";");
			break;
		case RP_COPY:
			for (long i = 0; i < I.n; i++) ln(wr(I.out, I.p[0] + i) + " = " + rd(I.a, I.p[1] + i) + ";");
			break;
		default: break;
		}
		return true;
	}

	bool think(const Node &n)
	{
		const rp_ins &T = S.prog[n.ins];
		for (auto &c : n.pre)
			if (!node(c)) return false;
		const std::string k = itos(loops++), it = "it" + k, sv = "sv" + k, d = "d" + k, stop = "stop" + k;
		ln("{ // think loop");
		depth++;
		for (long i = 0; i < T.n; i++) ln(wr(T.out, i) + " = " + rd(T.a, i) + ";");
		ln("int " + it + " = 0;");
		const bool halt = T.p[3] != INT_MIN;
		if (halt) ln(fx ? "int " + sv + " = 65536;" : "float " + sv + " = 1.0f;");
		ln("for (;;) {");
		depth++;
		for (auto &c : n.body)
			if (!node(c)) return false;
		ln(it + "++;");
		const int y = T.p[0];
		ln(fx ? "int " + d + " = 0;" : "float " + d + " = 0.0f;");
		for (long i = 0; i < T.n; i++) {
			if (fx) ln("{ const int e = tgrd::absq(tgrd::subq(" + rd(y, i) + ", " + rd(T.out, i) + ")); " + d + " = e > " + d + " ? e : " + d + "; }");
			else ln("{ const float e = fabsf(" + rd(y, i) + " - " + rd(T.out, i) + "); if (e > " + d + ") " + d + " = e; }");
		}
		for (long i = 0; i < T.n; i++) ln(wr(T.out, i) + " = " + rd(y, i) + ";");
		ln("bool " + stop + " = false;");
		if (fx) {
			if (T.p[2] >= 0) ln("if (" + d + " <= " + ilit(T.p[7]) + ") " + stop + " = true;");
		} else {
			float eps;
			memcpy(&eps, &T.p[2], 4);
			if (eps >= 0.0f) ln("if (" + d + " <= " + flit(eps) + ") " + stop + " = true;");
		}
		if (halt) {
			const std::string h = rd(T.p[3], 0);
			if (fx) {
				ln("if (!" + stop + ") { const int p = " + h + " < 0 ? 0 : " + h + " > 65536 ? 65536 : " + h + "; " + sv + " = tgrd::fmulq(" + sv +
				   ", 65536 - p); if (65536 - " + sv + " > " + ilit(T.p[8]) + ") " + stop + " = true; }");
			} else {
				float thr;
				memcpy(&thr, &T.p[4], 4);
				ln("if (!" + stop + ") { const float p = " + h + "; " + sv + " *= 1.0f - (p < 0.0f ? 0.0f : p > 1.0f ? 1.0f : p); if (1.0f - " + sv +
				   " > " + flit(thr) + ") " + stop + " = true; }");
			}
		}
		ln("if (" + stop + " || " + it + " >= " + itos(T.p[1]) + ") break;");
		depth--;
		ln("}");
		ln("if (steps) steps[row * " + itos(S.nthink) + " + " + itos(T.p[5]) + "] = " + it + ";");
		depth--;
		ln("}");
		return true;
	}

	bool node(const Node &n) { return S.prog[n.ins].kind == RP_THINK ? think(n) : ins(S.prog[n.ins]); }
};

// a header's text for inclusion in one translation unit: no include guard, no local includes
std::string inline_text(const char *text)
{
	std::string s(text), r;
	size_t i = 0;
	while (i < s.size()) {
		size_t e = s.find('\n', i);
		if (e == std::string::npos) e = s.size();
		std::string l = s.substr(i, e - i);
		if (l.rfind("#pragma once", 0) != 0 && l.rfind("#include \"", 0) != 0) r += l + "\n";
		i = e + 1;
	}
	return r;
}

} // namespace

bool rp_emit(const rp_source &S, const char *kernel, bool launcher, std::string &src, std::string &why, rp_emit_stats *st)
{
	if (S.arena > MAX_SLOTS) {
		why = "the arena has more slots than registers hold";
		return false;
	}
	std::vector<Node> top;
	int pc = 0;
	if (!parse(S, pc, -1, top, why)) return false;
	long hoisted = 0;
	for (auto &n : top)
		if (S.prog[n.ins].kind == RP_THINK) hoist(S, n, hoisted);
	Gen g(S);
	g.ln("const T *src = in + row * " + itos(S.per) + ";");
	for (long i = 0; i < S.per; i++) g.ln(g.wr(S.in_slot, i) + " = src[" + itos(i) + "];");
	for (auto &n : top)
		if (!g.node(n)) {
			why = "the program has more multiply-add terms than the compiled form takes";
			return false;
		}
	g.ln("T *dst = out + row * " + itos(S.nout) + ";");
	for (long i = 0; i < S.nout; i++) g.ln("dst[" + itos(i) + "] = " + g.rd(S.out_ref, i) + ";");

	const char *T = S.fixed ? "int" : "float";
	std::string h = "// Row program compiled for one model: one lane per batch row, values in registers.\n";
	h += inline_text(DEVMATH_TEXT);
	h += inline_text(ROWDEV_TEXT);
	h += "\nextern \"C\" __global__ __launch_bounds__(256) void " + std::string(kernel) + "(const " + T + " *__restrict__ in, " + T +
	     " *__restrict__ out, int *__restrict__ steps, int rows)\n{\n";
	h += "\ttypedef " + std::string(T) + " T;\n";
	h += "\tconst long row = (long)blockIdx.x * 256 + threadIdx.x;\n\tif (row >= rows) return;\n";
	long nslots = 0;
	std::string decl;
	for (long s = 0; s < S.arena; s++) {
		if (!g.used[s]) continue;
		decl += (nslots % 16 ? ", v" : (nslots ? ";\n\tT v" : "\tT v")) + itos(s) + " = 0";
		nslots++;
	}
	if (nslots) h += decl + ";\n";
	src = h + g.out + "}\n";
	if (launcher) { // TG_UNIT_KERNEL_ONLY leaves it out (a build of the kernel alone)
		src += "\n#ifndef TG_UNIT_KERNEL_ONLY\nextern \"C\" int " + std::string(kernel) + "_batch(const void *d_in, int rows, void *d_out, int *d_steps, hipStream_t st)\n{\n";
		src += "\tif (rows <= 0) return 0;\n";
		src += "\thipLaunchKernelGGL(" + std::string(kernel) + ", dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, st, (const " + T +
		       " *)d_in, (" + T + " *)d_out, d_steps, rows);\n";
		src += "\treturn hipGetLastError() == hipSuccess ? 0 : -1;\n}\n#endif\n";
	}
	if (st) {
		st->hoisted = hoisted;
		st->terms = g.terms;
		st->slots = nslots;
	}
	return true;
}
