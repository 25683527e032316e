// KV-cache greedy decoder for models in the Qwen3 importer's layout
// (examples/qwen3/import.py:46-130: per-head projections Wq_l_h, Wk_l_j,
// Wv_l_j, Wo_l_h, SwiGLU Wg_l / Wu_l / Wd_l, RMSNorm gains ln1_l, ln2_l,
// qn_l, kn_l, lnf, RoPE by a rotation matrix Rot, embedding E, LM head LM).
// The reference runs such a model at a fixed length only; it has no cache
// (the importer bakes the sequence length). This decoder runs the same graph
// over a chunk of positions at a time: a prompt of T0 tokens per sequence
// (prefill), then one token per sequence per step, keeping every layer's k and
// v in a cache. Every kernel is the one the layer executor uses for the same
// instruction (or, for one step's attention, one that keeps the same
// operations and order), each row depends only on itself, and the masked
// keys of the fixed-length graph contribute exact zeros. A step's logits
// therefore equal the fixed-length forward's at that position, bit for bit,
// for finite activations.
#include "tg_hip.h"
#include "tg_kern.h"
#include "tgm.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

const tgm_module *tgh_prog_module(const tg_hip_prog *p);
hipStream_t tgh_prog_stream(const tg_hip_prog *p);
void tgh_set_error(const char *msg);

struct tg_hip_dec {
	const tg_hip_prog *p = nullptr;
	hipStream_t st = nullptr;
	int L = 0, D = 0, NQ = 0, NKV = 0, HD = 0, FF = 0, V = 0;
	int S = 0, TP = 0, P = 0; // max sequences, max prompt, max positions
	float scale = 0.0f;
	std::vector<void *> allocs;
	std::vector<tgk_qweight> ws; // every packed weight, freed at the end
	// params
	const float *E = nullptr, *lnf = nullptr, *cosT = nullptr, *sinT = nullptr;
	std::vector<const float *> ln1, ln2, qkg;
	std::vector<int> wqkv, wgu, wd, wo; // indices into ws (wo: L x NQ)
	std::vector<const int *> wo_codes;  // per layer: all heads' output projections for a step, int32 [NQ][HD/4][D]
	std::vector<const float *> wo_scales; // per layer: [NQ][D]
	int wrot = -1, wlm = -1;
	// cache and work buffers
	float *K = nullptr, *Vc = nullptr;
	long kv_seq = 0;
	float *ids = nullptr, *h = nullptr, *n = nullptr, *qkv = nullptr, *hq = nullptr, *rt = nullptr;
	float *qr = nullptr, *att = nullptr, *wout = nullptr, *gu = nullptr, *act = nullptr, *dbuf = nullptr;
	float *sc = nullptr, *lastn = nullptr, *logits = nullptr;
	float *am_v = nullptr; // argmax workspace: TGK_AM_PARTS per sequence
	int *am_i = nullptr;
	void *scratch = nullptr;
	size_t scratch_bytes = 0;
};

namespace {

bool err(const char *fmt, const char *a = "", long b = 0)
{
	char buf[512];
	snprintf(buf, sizeof buf, fmt, a, b);
	tgh_set_error(buf);
	return false;
}

bool hip_ok(hipError_t e, const char *what)
{
	if (e == hipSuccess) return true;
	char buf[256];
	snprintf(buf, sizeof buf, "%s: %s", what, hipGetErrorString(e));
	tgh_set_error(buf);
	return false;
}

int find(const tgm_module *m, const std::string &name)
{
	for (int v = 0; v < m->nval; v++)
		if (m->val[v].kind == TGM_PARAM && m->val[v].name && name == m->val[v].name) return v;
	return -1;
}

std::string nm(const char *f, int a, int b = -1)
{
	char buf[64];
	if (b < 0) snprintf(buf, sizeof buf, f, a);
	else snprintf(buf, sizeof buf, f, a, b);
	return buf;
}

template <class T> bool alloc(tg_hip_dec *d, T **p, size_t n)
{
	void *q = nullptr;
	if (!hip_ok(hipMalloc(&q, n * sizeof(T) + 256), "decoder memory")) return false;
	d->allocs.push_back(q);
	*p = (T *)q;
	return true;
}

bool upload(tg_hip_dec *d, const float **dst, const float *src, size_t n)
{
	float *q;
	if (!alloc(d, &q, n)) return false;
	*dst = q;
	return hip_ok(hipMemcpyAsync(q, src, n * sizeof(float), hipMemcpyHostToDevice, d->st), "decoder upload");
}

// one layer's per-head output projections W_h [HD][D] (axis-1 scales) as
// the step kernel's code words: int32 [NQ][HD/4][D], codes of k = 4 k4 .. 4 k4
// + 3 in bytes 0 .. 3 of word (h, k4, c); scales [NQ][D]
bool pack_heads(tg_hip_dec *d, const tgm_module *m, const std::vector<int> &vs, const int **codes, const float **scales)
{
	const int HD = d->HD, D = d->D, NQ = (int)vs.size();
	std::vector<int> w((size_t)NQ * (HD / 4) * D, 0);
	std::vector<float> sc((size_t)NQ * D);
	for (int h = 0; h < NQ; h++) {
		const tgm_value &x = m->val[vs[(size_t)h]];
		if (x.sh.rank != 2 || x.sh.dim[0] != HD || x.sh.dim[1] != D || !x.qbits || x.qaxis != 1) return false;
		for (int k = 0; k < HD; k++)
			for (int c = 0; c < D; c++) {
				const unsigned b = (unsigned)(tgm_code(&x, (long)k * D + c) & 255);
				w[((size_t)h * (HD / 4) + k / 4) * D + c] |= (int)(b << (8 * (k % 4)));
			}
		memcpy(&sc[(size_t)h * D], x.qs, (size_t)D * sizeof(float));
	}
	int *q;
	if (!alloc(d, &q, w.size()) || !hip_ok(hipMemcpyAsync(q, w.data(), w.size() * sizeof(int), hipMemcpyHostToDevice, d->st), "decoder upload"))
		return false;
	*codes = q;
	return upload(d, scales, sc.data(), sc.size());
}

// pack params (each [K][C_i], quantized on axis 1, x @ W) concatenated along C
int pack_concat(tg_hip_dec *d, const tgm_module *m, const std::vector<int> &vs)
{
	const int K = m->val[vs[0]].sh.dim[0], bits = m->val[vs[0]].qbits;
	long C = 0;
	for (int v : vs) {
		const tgm_value &x = m->val[v];
		if (x.sh.rank != 2 || x.sh.dim[0] != K || x.qbits != bits || x.qaxis != 1) return -1;
		C += x.sh.dim[1];
	}
	std::vector<int8_t> codes((size_t)C * K);
	std::vector<float> scales((size_t)C);
	long c0 = 0;
	for (int v : vs) {
		const tgm_value &x = m->val[v];
		const int Ci = x.sh.dim[1];
		for (int c = 0; c < Ci; c++) {
			for (int k = 0; k < K; k++) codes[(size_t)(c0 + c) * K + k] = (int8_t)tgm_code(&x, (long)k * Ci + c);
			scales[(size_t)(c0 + c)] = x.qs[c];
		}
		c0 += Ci;
	}
	tgk_qweight w;
	if (tgk_qweight_pack_i8(&w, codes.data(), scales.data(), bits, (int)C, K, d->st)) return -1;
	d->ws.push_back(w);
	return (int)d->ws.size() - 1;
}

// o[rows][C] (row stride orr) = x[rows][K] (row stride xr) @ W, through the
// digit kernel and the matrix-core GEMM; ni inner rows of xj per batch row
bool gemm(tg_hip_dec *d, int wi, const float *x, long xr, int ni, long xj, int rows, float *o, long orr, long oj)
{
	tgk_qgemm_args a;
	memset(&a, 0, sizeof a);
	a.w = &d->ws[(size_t)wi];
	a.x = x;
	a.xr = xr, a.xj = xj, a.xk = 1, a.ni = ni;
	a.o = o;
	a.orr = orr, a.oc = 1, a.oj = oj;
	a.M = rows * ni;
	tgk_qgemm(d->st, &a, d->scratch);
	return true;
}

// o[rows][C] = x @ W with the activation digits already written (by the
// fused norm and silu kernels) into the GEMM's digit area for these rows;
// `resolved`: the producer resolved its candidate rows (else the split pass runs first)
bool gemm_pre(tg_hip_dec *d, int wi, const float *x, long xr, int ni, long xj, int rows, float *o, long orr, long oj, bool resolved)
{
	tgk_qgemm_args a;
	memset(&a, 0, sizeof a);
	a.w = &d->ws[(size_t)wi];
	a.x = x;
	a.xr = xr, a.xj = xj, a.xk = 1, a.ni = ni;
	a.o = o;
	a.orr = orr, a.oc = 1, a.oj = oj;
	a.M = rows * ni;
	if (!resolved) tgk_qgemm_split(d->st, &a, d->scratch); // the producer's candidate rows resolved
	tgk_qgemm_mfma(d->st, &a, d->scratch);
	return true;
}

// the graph's rmsnorm-then-gain of token rows, fused with the update of h
// before it (mode 1: h += add; mode 2: h += the heads' output projections in
// order) and the activation digits of weight wi's GEMM
bool norm(tg_hip_dec *d, int mode, float *h, long hs, int rows, const float *add, long adds, const float *g, float *out, int wi)
{
	tgk_dec_norm_args a;
	memset(&a, 0, sizeof a);
	a.h = h, a.hs = hs, a.mode = mode, a.add = add, a.adds = adds;
	a.o = d->wout, a.ohead = (long)rows * d->D, a.nh = d->NQ;
	a.g = g, a.out = out, a.outs = d->D, a.D = d->D, a.Kp = d->ws[(size_t)wi].Kp, a.rows = rows;
	a.q = tgk_qgemm_digit_area(d->scratch, rows, a.Kp);
	return tgk_dec_norm(d->st, &a);
}

// the graph over positions p0 .. p0 + T0 - 1 of S sequences, token ids in
// d->ids ([S][T0] f32); logits of the chunk's last position into d->logits
bool forward(tg_hip_dec *d, int S, int T0, int p0)
{
	const int rows = S * T0, NH = d->NQ + d->NKV, GRP = d->NQ / d->NKV;
	const long ctot = (long)(d->NQ + 2 * d->NKV) * d->HD, qk = (long)NH * d->HD, D = d->D;
	hipStream_t st = d->st;
	tgk_take(st, d->h, (long)T0 * D, tgk_opd{ d->E, 0 }, tgk_opd{ d->ids, T0 }, T0, d->V, d->D, S);
	for (int l = 0; l < d->L; l++) {
		const long kv_layer = (long)l * d->S * d->kv_seq; // the cache is layer-major: [layer][sequence][KV head][position][HD]
		// h (plus the previous layer's MLP output), rmsnorm * ln1, q k v projections
		bool res = norm(d, l == 0 ? 0 : 1, d->h, D, rows, d->dbuf, D, d->ln1[(size_t)l], d->n, d->wqkv[(size_t)l]);
		gemm_pre(d, d->wqkv[(size_t)l], d->n, D, 1, 0, rows, d->qkv, ctot, 0, res);
		tgk_dec_hnorm_args hn; // per-head rmsnorm * gain of the q and k heads, then the rotation matmul
		hn.x = d->qkv, hn.xs = ctot, hn.g = d->qkg[(size_t)l], hn.out = d->hq;
		hn.NH = NH, hn.HD = d->HD, hn.Kp = d->ws[(size_t)d->wrot].Kp, hn.rows = rows;
		hn.q = tgk_qgemm_digit_area(d->scratch, rows * NH, hn.Kp);
		res = tgk_dec_hnorm(st, &hn);
		gemm_pre(d, d->wrot, d->hq, qk, NH, d->HD, rows, d->rt, qk, d->HD, res);
		tgk_dec_rope_args r;
		r.hq = d->hq, r.rt = d->rt, r.qkv = d->qkv, r.ctot = ctot, r.cosT = d->cosT, r.sinT = d->sinT;
		r.qr = d->qr, r.K = d->K, r.V = d->Vc, r.kv_seq = d->kv_seq, r.kv_layer = kv_layer;
		r.T0 = T0, r.p0 = p0, r.NQ = d->NQ, r.NKV = d->NKV, r.HD = d->HD, r.P = d->P;
		tgk_dec_rope(st, &r, rows);
		if (T0 == 1) {
			tgk_dec_attn_args a;
			a.qr = d->qr, a.K = d->K, a.V = d->Vc, a.att = d->att, a.kv_seq = d->kv_seq, a.kv_layer = kv_layer;
			a.NQ = d->NQ, a.NKV = d->NKV, a.HD = d->HD, a.P = d->P, a.p = p0, a.scale = d->scale;
			tgk_dec_attn(st, &a, S);
		} else { // a prompt from position 0: per head, the graph's products, scale, mask and softmax (causal)
			for (int hh = 0; hh < d->NQ; hh++) {
				const int j = hh / GRP;
				tgk_mm m;
				memset(&m, 0, sizeof m);
				m.g = 1, m.m = T0, m.k = d->HD, m.n = T0, m.causal = 1;
				m.a = tgk_opd{ d->qr + (long)hh * d->HD, (long)T0 * d->NQ * d->HD }, m.ai = (long)d->NQ * d->HD, m.ap = 1;
				m.b = tgk_opd{ d->K + kv_layer + (long)j * d->P * d->HD, d->kv_seq }, m.bp = 1, m.bj = d->HD;
				m.o = d->sc, m.ors = (long)T0 * T0, m.oi = T0, m.oj = 1;
				tgk_matmul_exact(st, &m, S);
				tgk_dec_causal_softmax(st, d->sc, T0, (long)S * T0, d->scale);
				memset(&m, 0, sizeof m);
				m.g = 1, m.m = T0, m.k = T0, m.n = d->HD, m.causal = 2;
				m.a = tgk_opd{ d->sc, (long)T0 * T0 }, m.ai = T0, m.ap = 1;
				m.b = tgk_opd{ d->Vc + kv_layer + (long)j * d->P * d->HD, d->kv_seq }, m.bp = d->HD, m.bj = 1;
				m.o = d->att + (long)hh * d->HD, m.ors = (long)T0 * d->NQ * d->HD, m.oi = (long)d->NQ * d->HD, m.oj = 1;
				tgk_matmul_exact(st, &m, S);
			}
		}
		// a step: all heads in one launch, the same values (heads of at most TGK_REFLOOP_K take the
		// reference's loop, as every short product does: the per-head products below)
		if (T0 == 1 && d->HD > TGK_REFLOOP_K && tgk_dec_wo_lds(rows, d->HD) <= 65536)
			tgk_dec_wo(st, d->att, d->wo_codes[(size_t)l], d->wo_scales[(size_t)l], d->wout, rows, d->NQ, d->HD, d->D);
		else
			for (int hh = 0; hh < d->NQ; hh++)
				gemm(d, d->wo[(size_t)l * d->NQ + hh], d->att + (long)hh * d->HD, (long)d->NQ * d->HD, 1, 0, rows,
				     d->wout + (long)hh * rows * D, D, 0);
		// h + the heads' output projections (in head order), rmsnorm * ln2, gate and up projections
		res = norm(d, 2, d->h, D, rows, nullptr, 0, d->ln2[(size_t)l], d->n, d->wgu[(size_t)l]);
		gemm_pre(d, d->wgu[(size_t)l], d->n, D, 1, 0, rows, d->gu, 2L * d->FF, 0, res);
		if (rows >= TGK_DEC_SILU_FUSED_MAX) { // a prompt's many rows: act = silu(g) * u streamed, the down projection's own digits
			tgk_dec_silu_mul(st, d->gu, 2L * d->FF, d->act, d->FF, rows);
			gemm(d, d->wd[(size_t)l], d->act, d->FF, 1, 0, rows, d->dbuf, D, 0);
		} else {
			tgk_dec_silu_args sa; // act = silu(g) * u and its digits, then the down projection
			sa.gu = d->gu, sa.gus = 2L * d->FF, sa.out = d->act, sa.FF = d->FF, sa.Kp = d->ws[(size_t)d->wd[(size_t)l]].Kp;
			sa.rows = rows;
			sa.q = tgk_qgemm_digit_area(d->scratch, rows, sa.Kp);
			res = tgk_dec_silu(st, &sa);
			gemm_pre(d, d->wd[(size_t)l], d->act, d->FF, 1, 0, rows, d->dbuf, D, 0, res);
		}
	}
	// the last position of each sequence: h + the last MLP output, rmsnorm * lnf, LM head
	const bool res = norm(d, 1, d->h + (long)(T0 - 1) * D, (long)T0 * D, S, d->dbuf + (long)(T0 - 1) * D, (long)T0 * D, d->lnf, d->lastn,
			      d->wlm);
	gemm_pre(d, d->wlm, d->lastn, D, 1, 0, S, d->logits, d->V, 0, res);
	return hip_ok(hipGetLastError(), "decoder launch");
}

bool build(tg_hip_dec *d)
{
	const tgm_module *m = tgh_prog_module(d->p);
	const int vE = find(m, "E"), vLM = find(m, "LM"), vRot = find(m, "Rot"), vlnf = find(m, "lnf");
	const int vcos = find(m, "rope_cos"), vsin = find(m, "rope_sin");
	if (vE < 0 || vLM < 0 || vRot < 0 || vlnf < 0) return err("decoder: the model lacks E, LM, Rot or lnf (the Qwen3 importer's layout)");
	if (vcos < 0 || vsin < 0) return err("decoder: the model lacks rope_cos / rope_sin tables (one row per position)");
	d->V = m->val[vE].sh.dim[0], d->D = m->val[vE].sh.dim[1];
	while (find(m, nm("Wd_%d", d->L)) >= 0) d->L++;
	while (find(m, nm("Wq_0_%d", d->NQ)) >= 0) d->NQ++;
	while (find(m, nm("Wk_0_%d", d->NKV)) >= 0) d->NKV++;
	if (!d->L || !d->NQ || !d->NKV || d->NQ % d->NKV) return err("decoder: no layers or heads in the importer's naming");
	d->HD = m->val[find(m, "Wq_0_0")].sh.dim[1];
	d->FF = m->val[find(m, "Wg_0")].sh.dim[1];
	// one step's attention block: the scores of all positions in LDS; 1, 2, 4 or 8 query heads per KV head
	const int grp = d->NQ / d->NKV;
	if ((grp != 1 && grp != 2 && grp != 4 && grp != 8) || d->HD % 16 || d->HD > 256)
		return err("decoder: needs 1, 2, 4 or 8 query heads per KV head and a head size that is a multiple of 16, at most 256%s", "");
	if (d->D > TGK_DEC_NORM_MAX) return err("decoder: a model width above %s%ld", "", TGK_DEC_NORM_MAX);
	if (tgk_dec_attn_lds(grp, d->HD, d->P) > 65536) return err("decoder: %s%ld positions do not fit one step's attention (LDS)", "", d->P);
	if (m->val[vcos].sh.rank != 2 || m->val[vcos].sh.dim[1] != d->HD || m->val[vcos].sh.dim[0] < d->P)
		return err("decoder: rope tables need %s%ld rows", "", d->P);
	d->scale = 0.0f; // the graph's attention scale: its first constant (the importer writes 1/sqrt(HD) first)
	for (int i = 0; i < m->top.len && d->scale == 0.0f; i++)
		if (m->top.v[i].op == TGM_CONST) d->scale = m->top.v[i].k;
	if (d->scale == 0.0f) return err("decoder: no attention scale constant");
	d->st = tgh_prog_stream(d->p);
	const long HD = d->HD, NH = d->NQ + d->NKV, ctot = (long)(d->NQ + 2 * d->NKV) * HD;
	// params
	if (!upload(d, &d->E, m->val[vE].data, (size_t)m->val[vE].n) || !upload(d, &d->lnf, m->val[vlnf].data, (size_t)d->D)) return false;
	std::vector<float> tab((size_t)d->P * HD);
	memcpy(tab.data(), m->val[vcos].data, tab.size() * sizeof(float));
	if (!upload(d, &d->cosT, tab.data(), tab.size())) return false;
	memcpy(tab.data(), m->val[vsin].data, tab.size() * sizeof(float));
	if (!upload(d, &d->sinT, tab.data(), tab.size())) return false;
	d->ln1.resize((size_t)d->L), d->ln2.resize((size_t)d->L), d->qkg.resize((size_t)d->L);
	for (int l = 0; l < d->L; l++) {
		const int a = find(m, nm("ln1_%d", l)), b = find(m, nm("ln2_%d", l)), q = find(m, nm("qn_%d", l)), k = find(m, nm("kn_%d", l));
		if (a < 0 || b < 0 || q < 0 || k < 0) return err("decoder: layer %s%ld lacks a norm gain", "", l);
		std::vector<float> g((size_t)NH * HD); // the q heads' gain NQ times, then the k heads' NKV times
		for (int h = 0; h < NH; h++) memcpy(&g[(size_t)h * HD], m->val[h < d->NQ ? q : k].data, (size_t)HD * sizeof(float));
		if (!upload(d, &d->ln1[(size_t)l], m->val[a].data, (size_t)d->D) || !upload(d, &d->ln2[(size_t)l], m->val[b].data, (size_t)d->D) ||
		    !upload(d, &d->qkg[(size_t)l], g.data(), g.size()))
			return false;
		std::vector<int> qkv;
		for (int h = 0; h < d->NQ; h++) qkv.push_back(find(m, nm("Wq_%d_%d", l, h)));
		for (int j = 0; j < d->NKV; j++) qkv.push_back(find(m, nm("Wk_%d_%d", l, j)));
		for (int j = 0; j < d->NKV; j++) qkv.push_back(find(m, nm("Wv_%d_%d", l, j)));
		std::vector<int> gu{ find(m, nm("Wg_%d", l)), find(m, nm("Wu_%d", l)) };
		for (int v : qkv)
			if (v < 0 || !m->val[v].qbits) return err("decoder: layer %s%ld lacks a quantized projection", "", l);
		if (gu[0] < 0 || gu[1] < 0 || find(m, nm("Wd_%d", l)) < 0) return err("decoder: layer %s%ld lacks its MLP", "", l);
		const int i1 = pack_concat(d, m, qkv), i2 = pack_concat(d, m, gu), i3 = pack_concat(d, m, { find(m, nm("Wd_%d", l)) });
		if (i1 < 0 || i2 < 0 || i3 < 0) return err("decoder: cannot place layer %s%ld's weights", "", l);
		d->wqkv.push_back(i1), d->wgu.push_back(i2), d->wd.push_back(i3);
		std::vector<int> wo;
		for (int h = 0; h < d->NQ; h++) {
			const int v = find(m, nm("Wo_%d_%d", l, h));
			const int i = v < 0 ? -1 : pack_concat(d, m, { v });
			if (i < 0) return err("decoder: cannot place layer %s%ld's output projections", "", l);
			d->wo.push_back(i), wo.push_back(v);
		}
		const int *woc = nullptr;
		const float *wos = nullptr;
		if (!pack_heads(d, m, wo, &woc, &wos)) return err("decoder: cannot place layer %s%ld's output projections", "", l);
		d->wo_codes.push_back(woc), d->wo_scales.push_back(wos);
	}
	d->wrot = pack_concat(d, m, { vRot });
	d->wlm = pack_concat(d, m, { vLM });
	if (d->wrot < 0 || d->wlm < 0) return err("decoder: cannot place Rot or the LM head");
	// cache and buffers
	const long rows = (long)d->S * d->TP;
	d->kv_seq = (long)d->NKV * d->P * HD; // one sequence's K (or V) of one layer; a layer holds S of them
	if (!alloc(d, &d->K, (size_t)(d->L * d->S * d->kv_seq)) || !alloc(d, &d->Vc, (size_t)(d->L * d->S * d->kv_seq)) || !alloc(d, &d->ids, (size_t)rows) ||
	    !alloc(d, &d->h, (size_t)(rows * d->D)) ||
	    !alloc(d, &d->n, (size_t)(rows * d->D)) || !alloc(d, &d->qkv, (size_t)(rows * ctot)) || !alloc(d, &d->hq, (size_t)(rows * NH * HD)) ||
	    !alloc(d, &d->rt, (size_t)(rows * NH * HD)) || !alloc(d, &d->qr, (size_t)(rows * d->NQ * HD)) ||
	    !alloc(d, &d->att, (size_t)(rows * d->NQ * HD)) || !alloc(d, &d->wout, (size_t)(rows * d->NQ * d->D)) ||
	    !alloc(d, &d->gu, (size_t)(rows * 2 * d->FF)) || !alloc(d, &d->act, (size_t)(rows * d->FF)) || !alloc(d, &d->dbuf, (size_t)(rows * d->D)) ||
	    !alloc(d, &d->sc, (size_t)((long)d->S * d->TP * d->TP)) ||
	    !alloc(d, &d->lastn, (size_t)((long)d->S * d->D)) || !alloc(d, &d->logits, (size_t)((long)d->S * d->V)) ||
	    !alloc(d, &d->am_v, (size_t)d->S * TGK_AM_PARTS) || !alloc(d, &d->am_i, (size_t)d->S * TGK_AM_PARTS))
		return false;
	size_t sb = 0;
	auto need = [&](long M, int wi) { sb = std::max(sb, tgk_qgemm_scratch((int)M, d->ws[(size_t)wi].Kp)); };
	need(rows, d->wqkv[0]), need(rows * NH, d->wrot), need(rows, d->wo[0]), need(rows, d->wgu[0]), need(rows, d->wd[0]), need(d->S, d->wlm);
	d->scratch_bytes = sb;
	return hip_ok(hipMalloc(&d->scratch, sb), "decoder scratch") && hip_ok(hipStreamSynchronize(d->st), "decoder upload");
}

} // namespace

extern "C" {

tg_hip_dec *tg_hip_dec_create(const tg_hip_prog *p, int max_seqs, int max_prompt, int max_len)
{
	if (!p || max_seqs <= 0 || max_prompt <= 0 || max_len < max_prompt) {
		err("tg_hip_dec_create: bad arguments");
		return nullptr;
	}
	if (max_prompt > TGK_DEC_PROMPT_MAX) {
		err("tg_hip_dec_create: prompts of at most %s%ld tokens", "", TGK_DEC_PROMPT_MAX);
		return nullptr;
	}
	tg_hip_dec *d = new tg_hip_dec;
	d->p = p, d->S = max_seqs, d->TP = max_prompt, d->P = max_len;
	if (!build(d)) {
		tg_hip_dec_free(d);
		return nullptr;
	}
	return d;
}

int tg_hip_dec_generate(tg_hip_dec *d, const float *d_prompt, int seqs, int prompt_len, int steps, int *d_tokens, float *d_logits)
{
	if (!d || !d_prompt || seqs <= 0 || seqs > d->S || prompt_len <= 0 || prompt_len > d->TP || steps <= 0 ||
	    prompt_len + steps - 1 > d->P) {
		err("tg_hip_dec_generate: bad arguments (sequences, prompt length or steps beyond the decoder's sizes)");
		return -1;
	}
	if (!hip_ok(hipMemcpyAsync(d->ids, d_prompt, (size_t)seqs * prompt_len * sizeof(float), hipMemcpyDeviceToDevice, d->st), "prompt"))
		return -1;
	for (int s = 0; s < steps; s++) {
		const bool first = s == 0;
		if (!forward(d, seqs, first ? prompt_len : 1, first ? 0 : prompt_len + s - 1)) return -1;
		if (d_logits &&
		    !hip_ok(hipMemcpyAsync(d_logits + (size_t)s * seqs * d->V, d->logits, (size_t)seqs * d->V * sizeof(float),
					   hipMemcpyDeviceToDevice, d->st),
			    "logits"))
			return -1;
		tgk_dec_argmax(d->st, d->logits, d->V, d->V, seqs, d->ids, d_tokens ? d_tokens + s : nullptr, steps, d->am_v, d->am_i);
	}
	return hip_ok(hipGetLastError(), "decoder") ? 0 : -1;
}

int tg_hip_dec_info(const tg_hip_dec *d, int *layers, int *vocab)
{
	if (!d) return -1;
	if (layers) *layers = d->L;
	if (vocab) *vocab = d->V;
	return 0;
}

void tg_hip_dec_free(tg_hip_dec *d)
{
	if (!d) return;
	if (d->st) (void)hipStreamSynchronize(d->st);
	for (tgk_qweight &w : d->ws) tgk_qweight_free(&w);
	for (void *q : d->allocs) (void)hipFree(q);
	if (d->scratch) (void)hipFree(d->scratch);
	delete d;
}

} // extern "C"
