// test_mirror.cpp -- the reference's MoE C++ API (include/hunyuan_moe_full.h) served by
// the GPU library, checked against the CPU oracle.  Built by build.py, run by
// tests/test_gpu_mirror.py on a GPU.  Prints one PASS/FAIL line per check and exits
// with the number of failures.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "hunyuan_model_moe.h"
#include "hunyuan_moe_full.h"
#include "hy_oracle.h"

static int g_fail = 0;

static void report(bool ok, const char* name, const std::string& detail = "") {
    printf("%s %s%s%s\n", ok ? "PASS" : "FAIL", name, detail.empty() ? "" : ": ", detail.c_str());
    fflush(stdout);
    if (!ok) g_fail++;
}

static std::vector<float> synth(uint64_t seed, uint32_t tensor, uint32_t expert, size_t n, float std) {
    std::vector<float> v(n);
    hyo_synth_fill(hyo_stream_key(seed, 0, tensor, expert), 0, n, std, v.data());
    return v;
}

static bool bits_equal(const float* a, const float* b, size_t n) { return memcmp(a, b, n * 4) == 0; }

static double rel_err(const float* a, const float* b, size_t n) {
    double m = 0, d = 0;
    for (size_t i = 0; i < n; i++) {
        m = std::fmax(m, std::fabs((double)b[i]));
        d = std::fmax(d, std::fabs((double)a[i] - b[i]));
    }
    return m > 0 ? d / m : d;
}

static std::string errs(const float* a, const float* b, size_t n) {
    char buf[64];
    snprintf(buf, sizeof(buf), "rel_err=%.3e", rel_err(a, b, n));
    return buf;
}

int main() {
    // ---------------------------------------------------------------- top-k / softmax
    {
        std::vector<float> x(64);
        bool ok = true;
        for (int rep = 0; rep < 20; rep++) {
            for (int i = 0; i < 64; i++) x[i] = (float)(((i * 37 + rep * 11) % 9) - 4) * 0.5f;  // many ties
            for (uint32_t k : {1u, 4u, 8u, 64u}) {
                std::vector<float> v(k), vr(k);
                std::vector<int32_t> id(k), idr(k);
                topk_f32(x.data(), 64, k, v.data(), id.data());
                hyo_topk_f32(x.data(), 64, k, vr.data(), idr.data());
                ok = ok && v == vr && id == idr;
            }
        }
        report(ok, "topk_f32 matches the reference insertion order (ties -> lower index)");
    }
    {
        std::vector<float> x = synth(1, 0, 0, 64, 3.0f), r = x;
        softmax_f32(x.data(), 64);
        hyo_softmax_f32(r.data(), 64);
        report(rel_err(x.data(), r.data(), 64) < 2e-6, "softmax_f32", errs(x.data(), r.data(), 64));
    }
    // ---------------------------------------------------------------- gating
    const uint32_t T = 37, E = 64, K = 8;
    std::vector<float> lg = synth(2, 0, 0, (size_t)T * E, 1.5f);
    {
        std::vector<float> w(T * K), wr(T * K);
        std::vector<int32_t> i(T * K), ir(T * K);
        topkgating_easy(lg.data(), T, E, K, w.data(), i.data());
        hyo_topkgating_easy(lg.data(), T, E, K, wr.data(), ir.data());
        report(i == ir && rel_err(w.data(), wr.data(), w.size()) < 2e-6, "topkgating_easy",
               errs(w.data(), wr.data(), w.size()));
    }
    {
        MoERoutingConfig cfg;
        MoEGateOutput g;
        g.alloc(T, E, K, 1, true);  // deliberately too small: topkgating_full sizes its own capacity
        topkgating_full(lg.data(), T, cfg, g);
        hyo_routing_cfg rc;
        hyo_routing_cfg_default(&rc);
        hyo_gate_full ref;
        hyo_topkgating_full(lg.data(), T, &rc, &ref);
        const size_t n = (size_t)T * E * ref.capacity;
        bool ok = g.expert_capacity == ref.capacity && g.exp_capacity_rate == ref.exp_capacity_rate &&
                  memcmp(g.exp_counts, ref.exp_counts, E * 4) == 0;
        for (size_t i = 0; ok && i < n; i++) ok = (g.dispatch_mask[i] ? 1 : 0) == ref.dispatch_mask[i];
        const double ecw = rel_err(g.combine_weights, ref.combine_weights, n);
        const double epr = rel_err(g.router_probs, ref.router_probs, (size_t)T * E);
        report(ok && ecw < 2e-6 && epr < 2e-6, "topkgating_full (mask, slots, counts, capacity exact)",
               "cw " + errs(g.combine_weights, ref.combine_weights, n));
        hyo_gate_full_free(&ref);
        bool threw = false;
        try {
            MoERoutingConfig bad;
            bad.drop_tokens = true;
            topkgating_full(lg.data(), T, bad, g);
        } catch (const hy::Error& e) {
            threw = e.code == HY_ERR_UNSUPPORTED;
        }
        report(threw, "topkgating_full rejects token dropping on the GPU path");
    }
    // ---------------------------------------------------------------- einsum dispatch / combine
    {
        const uint32_t Tt = 9, H = 96, Ee = 6, C = 4;
        std::vector<float> x = synth(3, 0, 0, (size_t)Tt * H, 1.0f);
        std::vector<uint8_t> m8((size_t)Tt * Ee * C);
        bool m[9 * 6 * 4];
        for (size_t i = 0; i < m8.size(); i++) m[i] = m8[i] = ((i * 7 + 3) % 5) == 0;
        std::vector<float> d((size_t)Ee * C * H), dr(d.size());
        einsum_dispatch(x.data(), Tt, H, m, Ee, C, d.data());
        hyo_einsum_dispatch(x.data(), Tt, H, m8.data(), Ee, C, dr.data());
        report(bits_equal(d.data(), dr.data(), d.size()), "einsum_dispatch bit-exact");
        std::vector<float> cw = synth(4, 0, 0, (size_t)Tt * Ee * C, 1.0f), eo = synth(5, 0, 0, d.size(), 1.0f);
        for (size_t i = 0; i < cw.size(); i++)
            if (!m8[i]) cw[i] = 0.0f;
        std::vector<float> o((size_t)Tt * H), orf(o.size());
        einsum_combine(cw.data(), eo.data(), Tt, H, Ee, C, o.data());
        hyo_einsum_combine(cw.data(), eo.data(), Tt, H, Ee, C, orf.data());
        report(bits_equal(o.data(), orf.data(), o.size()), "einsum_combine bit-exact");
    }
    // ---------------------------------------------------------------- layer forwards
    const uint32_t H = 256, I = 128, Ex = 16, Kx = 4, Tl = 21;
    std::vector<float> x = synth(6, 0, 0, (size_t)Tl * H, 1.0f);
    std::vector<float> wr = synth(6, 1, 0, (size_t)Ex * H, 0.1f);
    std::vector<float> gu = synth(6, 2, 0, (size_t)Ex * 2 * I * H, 0.05f), dn = synth(6, 3, 0, (size_t)Ex * H * I, 0.05f);
    std::vector<float> sgu = synth(6, 2, Ex, (size_t)2 * I * H, 0.05f), sdn = synth(6, 3, Ex, (size_t)H * I, 0.05f);
    MoERoutingConfig rcfg;
    rcfg.num_experts = Ex;
    rcfg.moe_topk = Kx;
    {
        std::vector<float> out((size_t)Tl * H), ref(out.size()), q(out.size());
        moe_forward_full(x.data(), Tl, H, wr.data(), sgu.data(), sdn.data(), gu.data(), dn.data(), Ex, I, rcfg,
                         out.data());
        hyo_routing_cfg rc;
        hyo_routing_cfg_default(&rc);
        rc.num_experts = Ex;
        rc.moe_topk = Kx;
        hyo_moe_forward_full(x.data(), Tl, H, wr.data(), sgu.data(), sdn.data(), gu.data(), dn.data(), Ex, I, &rc,
                             ref.data());
        hyo_qlayer L{H, I, Ex, Kx, HYO_F32, 1, 1.0f, wr.data(), sgu.data(), sdn.data(), gu.data(), dn.data()};
        hyo_moe_forward_q(&L, x.data(), Tl, q.data(), nullptr, nullptr, nullptr, 1);
        report(bits_equal(out.data(), q.data(), out.size()), "moe_forward_full F32 == q semantics bit-exact");
        report(rel_err(out.data(), ref.data(), out.size()) < 1e-4, "moe_forward_full F32 vs reference semantics",
               errs(out.data(), ref.data(), out.size()));
    }
    for (int wt : {HYO_Q8_0, HYO_Q4_0}) {
        const size_t rb_h = hyo_type_row_bytes(wt, H), rb_i = hyo_type_row_bytes(wt, I);
        std::vector<uint8_t> qgu((size_t)Ex * 2 * I * rb_h), qdn((size_t)Ex * H * rb_i), qsgu(2 * I * rb_h),
            qsdn(H * rb_i);
        auto quant = (wt == HYO_Q8_0) ? hyo_quantize_row_q8_0 : hyo_quantize_row_q4_0;
        quant(gu.data(), qgu.data(), gu.size());
        quant(dn.data(), qdn.data(), dn.size());
        quant(sgu.data(), qsgu.data(), sgu.size());
        quant(sdn.data(), qsdn.data(), sdn.size());
        std::vector<float> out((size_t)Tl * H), ref(out.size());
        moe_forward_full(x.data(), Tl, H, wr.data(), qsgu.data(), qsdn.data(), qgu.data(), qdn.data(), wt, Ex, I, rcfg,
                         out.data());
        hyo_qlayer L{H, I, Ex, Kx, wt, 1, 1.0f, wr.data(), qsgu.data(), qsdn.data(), qgu.data(), qdn.data()};
        hyo_moe_forward_q(&L, x.data(), Tl, ref.data(), nullptr, nullptr, nullptr, 1);
        report(bits_equal(out.data(), ref.data(), out.size()),
               wt == HYO_Q8_0 ? "moe_forward_full Q8_0 overload bit-exact" : "moe_forward_full Q4_0 overload bit-exact",
               errs(out.data(), ref.data(), out.size()));
    }
    {
        std::vector<float> out((size_t)Tl * H), ref(out.size());
        swiglu_ffn_f32(x.data(), sgu.data(), sdn.data(), out.data(), Tl, H, I);
        hyo_swiglu_ffn_f32(x.data(), sgu.data(), sdn.data(), ref.data(), Tl, H, I);
        report(rel_err(out.data(), ref.data(), out.size()) < 1e-4, "swiglu_ffn_f32", errs(out.data(), ref.data(), out.size()));
    }
    {
        MoEWeights w;
        w.num_experts = Ex;
        w.router_weight = wr;
        w.shared_gate_up = sgu;
        w.shared_down = sdn;
        w.experts.resize(Ex);
        for (uint32_t e = 0; e < Ex; e++) {
            w.experts[e].gate_up.assign(gu.begin() + (size_t)e * 2 * I * H, gu.begin() + (size_t)(e + 1) * 2 * I * H);
            w.experts[e].down.assign(dn.begin() + (size_t)e * H * I, dn.begin() + (size_t)(e + 1) * H * I);
        }
        HunyuanConfig cfg;
        cfg.hidden_size = H;
        cfg.moe_intermediate_size = I;
        cfg.moe_topk = Kx;
        std::vector<float> out((size_t)Tl * H), ref(out.size()), p((size_t)Tl * Ex), pr(p.size()), dw(Tl * Kx),
            dwr(dw.size());
        std::vector<int32_t> di(Tl * Kx), dir(di.size());
        moe_forward_cpu(x.data(), w, Tl, cfg, out.data(), p.data(), dw.data(), di.data());
        hyo_moe_forward_cpu(x.data(), wr.data(), sgu.data(), sdn.data(), gu.data(), dn.data(), Tl, H, Ex, I, Kx,
                            ref.data(), pr.data(), dwr.data(), dir.data());
        report(di == dir && rel_err(p.data(), pr.data(), p.size()) < 2e-6 && rel_err(dw.data(), dwr.data(), dw.size()) < 2e-6,
               "moe_forward_cpu debug router outputs");
        report(rel_err(out.data(), ref.data(), out.size()) < 1e-4, "moe_forward_cpu", errs(out.data(), ref.data(), out.size()));
    }
    {
        std::vector<float> w = synth(7, 0, 0, H, 1.0f), out((size_t)Tl * H), ref(out.size());
        rms_norm_f32(x.data(), w.data(), out.data(), Tl, H, 1e-5f);
        hyo_rms_norm_f32(x.data(), w.data(), ref.data(), Tl, H, 1e-5f);
        report(rel_err(out.data(), ref.data(), out.size()) < 1e-6, "rms_norm_f32", errs(out.data(), ref.data(), out.size()));
    }
    {
        bool threw = false;
        try {
            std::vector<float> out(100);
            moe_forward_full(x.data(), 1, 100, wr.data(), nullptr, nullptr, gu.data(), dn.data(), Ex, I, rcfg, out.data());
        } catch (const hy::Error& e) {
            threw = e.code == HY_ERR_INVALID;
        }
        report(threw, "moe_forward_full rejects a hidden size the kernels do not tile");
    }
    printf("%d failure(s)\n", g_fail);
    return g_fail;
}
