// test_mirror.cpp -- the reference's MoE C++ API (include/hunyuan_moe_full.h) served by
// the GPU library, checked against the CPU oracle.  Built by build.py, run by
// tests/test_gpu_mirror.py on a GPU.  Prints one PASS/FAIL line per check and exits
// with the number of failures.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "hunyuan_model_attn.h"
#include "hunyuan_model_moe.h"
#include "hunyuan_moe_full.h"
#include "hy_oracle.h"
#include "hy_oracle_attn.h"

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
    }
    // routing options: group-limited greedy, token dropping, the aux loss, alone and together
    for (int opt = 0; opt < 4; opt++) {
        const uint32_t To = 61, Eo = 16, Ko = 4;
        std::vector<float> lo = synth(40 + opt, 0, 0, (size_t)To * Eo, 1.5f);
        MoERoutingConfig cfg;
        cfg.num_experts = Eo;
        cfg.moe_topk = Ko;
        hyo_routing_cfg rc;
        hyo_routing_cfg_default(&rc);
        rc.num_experts = Eo;
        rc.moe_topk = Ko;
        if (opt == 0 || opt == 3) {
            cfg.group_limited_greedy = rc.group_limited_greedy = 1;
            cfg.n_group = rc.n_group = 4;
            cfg.topk_group = rc.topk_group = 2;
        }
        if (opt == 1 || opt == 3) {
            cfg.drop_tokens = rc.drop_tokens = 1;
            cfg.capacity_factor = rc.capacity_factor = 0.75f;
            cfg.min_capacity = rc.min_capacity = 3;
        }
        if (opt == 2 || opt == 3) cfg.compute_aux_loss = rc.compute_aux_loss = 1;
        MoEGateOutput g;
        topkgating_full(lo.data(), To, cfg, g);
        hyo_gate_full ref;
        hyo_topkgating_full(lo.data(), To, &rc, &ref);
        const size_t n = (size_t)To * Eo * ref.capacity;
        bool ok = g.expert_capacity == ref.capacity && g.exp_capacity_rate == ref.exp_capacity_rate &&
                  memcmp(g.exp_counts, ref.exp_counts, Eo * 4) == 0;
        size_t placed = 0;
        for (size_t i = 0; ok && i < n; i++) {
            ok = (g.dispatch_mask[i] ? 1 : 0) == ref.dispatch_mask[i];
            placed += ref.dispatch_mask[i] ? 1 : 0;
        }
        const double ecw = rel_err(g.combine_weights, ref.combine_weights, n);
        const double epr = rel_err(g.router_probs, ref.router_probs, (size_t)To * Eo);
        const double eaux = std::fabs((double)g.aux_loss - ref.aux_loss) / std::fmax(1e-30, std::fabs((double)ref.aux_loss));
        const bool aux_ok = rc.compute_aux_loss ? eaux < 2e-5 : g.aux_loss == 0.0f;
        const bool dropped = !rc.drop_tokens || placed < (size_t)To * Ko;  // the case does drop pairs
        static const char* names[] = {"topkgating_full group-limited greedy", "topkgating_full token dropping",
                                      "topkgating_full aux loss", "topkgating_full groups + dropping + aux loss"};
        char det[160];
        snprintf(det, sizeof(det), "cap %u/%u rate %g/%g cw %.2e probs %.2e aux %g/%g placed %zu", g.expert_capacity,
                 ref.capacity, g.exp_capacity_rate, ref.exp_capacity_rate, ecw, epr, g.aux_loss, ref.aux_loss, placed);
        report(ok && ecw < 2e-6 && epr < 2e-6 && aux_ok && dropped, names[opt], det);
        hyo_gate_full_free(&ref);
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
    // moe_forward_full with group-limited greedy and token dropping (F32 and Q8_0)
    {
        MoERoutingConfig oc = rcfg;
        oc.group_limited_greedy = true;
        oc.n_group = 4;
        oc.topk_group = 3;
        oc.drop_tokens = true;
        oc.capacity_factor = 0.5f;  // capacity max(4, (uint32)(0.5 * 4 * 21 / 16)) = 4 < 5.25 pairs per expert
        oc.min_capacity = 0;
        hyo_routing_cfg rc;
        hyo_routing_cfg_default(&rc);
        rc.num_experts = Ex;
        rc.moe_topk = Kx;
        rc.group_limited_greedy = 1;
        rc.n_group = 4;
        rc.topk_group = 3;
        rc.drop_tokens = 1;
        rc.capacity_factor = 0.5f;
        rc.min_capacity = 0;
        const uint32_t cap = hyo_drop_capacity(Tl, Ex, Kx, 0.5f, 0);
        std::vector<float> out((size_t)Tl * H), ref(out.size()), q(out.size());
        moe_forward_full(x.data(), Tl, H, wr.data(), sgu.data(), sdn.data(), gu.data(), dn.data(), Ex, I, oc, out.data());
        hyo_moe_forward_full(x.data(), Tl, H, wr.data(), sgu.data(), sdn.data(), gu.data(), dn.data(), Ex, I, &rc,
                             ref.data());
        hyo_qlayer L{H, I, Ex, Kx, HYO_F32, 1, 1.0f, wr.data(), sgu.data(), sdn.data(), gu.data(), dn.data(), 4, 3, cap};
        hyo_moe_forward_q(&L, x.data(), Tl, q.data(), nullptr, nullptr, nullptr, 1);
        report(bits_equal(out.data(), q.data(), out.size()), "moe_forward_full F32 groups + dropping == q semantics",
               errs(out.data(), q.data(), out.size()));
        report(rel_err(out.data(), ref.data(), out.size()) < 1e-4,
               "moe_forward_full F32 groups + dropping vs reference semantics", errs(out.data(), ref.data(), out.size()));
        const size_t rb_h = hyo_type_row_bytes(HYO_Q8_0, H), rb_i = hyo_type_row_bytes(HYO_Q8_0, I);
        std::vector<uint8_t> qgu((size_t)Ex * 2 * I * rb_h), qdn((size_t)Ex * H * rb_i), qsgu(2 * I * rb_h),
            qsdn(H * rb_i);
        hyo_quantize_row_q8_0(gu.data(), qgu.data(), gu.size());
        hyo_quantize_row_q8_0(dn.data(), qdn.data(), dn.size());
        hyo_quantize_row_q8_0(sgu.data(), qsgu.data(), sgu.size());
        hyo_quantize_row_q8_0(sdn.data(), qsdn.data(), sdn.size());
        moe_forward_full(x.data(), Tl, H, wr.data(), qsgu.data(), qsdn.data(), qgu.data(), qdn.data(), HYO_Q8_0, Ex, I,
                         oc, out.data());
        hyo_qlayer LQ{H, I, Ex, Kx, HYO_Q8_0, 1, 1.0f, wr.data(), qsgu.data(), qsdn.data(), qgu.data(), qdn.data(),
                      4, 3, cap};
        hyo_moe_forward_q(&LQ, x.data(), Tl, q.data(), nullptr, nullptr, nullptr, 1);
        report(bits_equal(out.data(), q.data(), out.size()), "moe_forward_full Q8_0 groups + dropping == q semantics",
               errs(out.data(), q.data(), out.size()));
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
    // ---------------------------------------------------------------- one expert per token (K = 1)
    // topkgating_full keeps p * routed_scaling_factor (src/hunyuan_moe_full.cpp:230 `norm_topk_prob
    // && K > 1`), so moe_forward_full does too; topkgating_easy and moe_forward_cpu renormalise to 1.
    for (float scale : {1.0f, 2.5f}) {
        MoERoutingConfig c1;
        c1.num_experts = E;
        c1.moe_topk = 1;
        c1.routed_scaling_factor = scale;
        MoEGateOutput g;
        topkgating_full(lg.data(), T, c1, g);
        hyo_routing_cfg rc;
        hyo_routing_cfg_default(&rc);
        rc.num_experts = E;
        rc.moe_topk = 1;
        rc.routed_scaling_factor = scale;
        hyo_gate_full ref;
        hyo_topkgating_full(lg.data(), T, &rc, &ref);
        const size_t n = (size_t)T * E * ref.capacity;
        bool ok = g.expert_capacity == ref.capacity && memcmp(g.exp_counts, ref.exp_counts, E * 4) == 0;
        for (size_t i = 0; ok && i < n; i++) ok = (g.dispatch_mask[i] ? 1 : 0) == ref.dispatch_mask[i];
        report(ok && rel_err(g.combine_weights, ref.combine_weights, n) < 2e-6,
               scale == 1.0f ? "topkgating_full K=1 keeps p (no renormalisation)"
                             : "topkgating_full K=1 keeps p * routed_scaling_factor",
               "cw " + errs(g.combine_weights, ref.combine_weights, n));
        hyo_gate_full_free(&ref);
    }
    {
        std::vector<float> w(T), wr(T);
        std::vector<int32_t> i(T), ir(T);
        topkgating_easy(lg.data(), T, E, 1, w.data(), i.data());
        hyo_topkgating_easy(lg.data(), T, E, 1, wr.data(), ir.data());
        bool ones = true;
        for (float v : w) ones = ones && v == 1.0f;
        report(i == ir && ones && bits_equal(w.data(), wr.data(), T), "topkgating_easy K=1 weights are exactly 1");
    }
    {
        MoERoutingConfig c1;
        c1.num_experts = Ex;
        c1.moe_topk = 1;
        c1.routed_scaling_factor = 1.5f;
        std::vector<float> out((size_t)Tl * H), ref(out.size()), q(out.size());
        moe_forward_full(x.data(), Tl, H, wr.data(), sgu.data(), sdn.data(), gu.data(), dn.data(), Ex, I, c1,
                         out.data());
        hyo_routing_cfg rc;
        hyo_routing_cfg_default(&rc);
        rc.num_experts = Ex;
        rc.moe_topk = 1;
        rc.routed_scaling_factor = 1.5f;
        hyo_moe_forward_full(x.data(), Tl, H, wr.data(), sgu.data(), sdn.data(), gu.data(), dn.data(), Ex, I, &rc,
                             ref.data());
        hyo_qlayer L{H, I, Ex, 1, HYO_F32, 1, 1.5f, wr.data(), sgu.data(), sdn.data(), gu.data(), dn.data()};
        hyo_moe_forward_q(&L, x.data(), Tl, q.data(), nullptr, nullptr, nullptr, 1);
        report(bits_equal(out.data(), q.data(), out.size()) && rel_err(out.data(), ref.data(), out.size()) < 1e-4,
               "moe_forward_full K=1 (p * scale) vs reference semantics", errs(out.data(), ref.data(), out.size()));

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
        cfg.moe_topk = 1;
        std::vector<float> oc(out.size()), rcpu(out.size()), dw(Tl), dwr(Tl);
        std::vector<int32_t> di(Tl), dir(Tl);
        moe_forward_cpu(x.data(), w, Tl, cfg, oc.data(), nullptr, dw.data(), di.data());
        hyo_moe_forward_cpu(x.data(), wr.data(), sgu.data(), sdn.data(), gu.data(), dn.data(), Tl, H, Ex, I, 1,
                            rcpu.data(), nullptr, dwr.data(), dir.data());
        bool ones = true;
        for (float v : dw) ones = ones && v == 1.0f;
        report(di == dir && ones && bits_equal(dw.data(), dwr.data(), Tl) &&
                   rel_err(oc.data(), rcpu.data(), oc.size()) < 1e-4,
               "moe_forward_cpu K=1 renormalises to weight 1", errs(oc.data(), rcpu.data(), oc.size()));
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
    // ---------------------------------------------------------------- attention half, decoder layer, backbone helpers
    {
        HunyuanConfig cfg;
        cfg.hidden_size = 256;
        cfg.num_attention_heads = 8;
        cfg.num_key_value_heads = 2;
        cfg.attention_head_dim = 64;
        cfg.moe_intermediate_size = 128;
        cfg.moe_topk = 2;
        cfg.compute_derived();
        const uint32_t Ha = 256, nh = 8, nkv = 2, hd = 64, Ta = 9, Ea = 8;
        const size_t nq = (size_t)nh * hd, nk = (size_t)nkv * hd;
        AttentionWeights aw;
        aw.qkv_weight = synth(30, 4, 0, (nq + 2 * nk) * Ha, 0.05f);
        aw.o_weight = synth(31, 5, 0, Ha * nq, 0.05f);
        aw.q_norm_weight = synth(32, 0, 0, hd, 0.2f);
        aw.k_norm_weight = synth(33, 0, 0, hd, 0.2f);
        for (auto& v : aw.q_norm_weight) v += 1.0f;
        for (auto& v : aw.k_norm_weight) v += 1.0f;
        std::vector<float> xa = synth(34, 0, 0, (size_t)Ta * Ha, 1.0f);
        std::vector<int> pos(Ta);
        for (uint32_t t = 0; t < Ta; t++) pos[t] = (int)(3 * t + 1);
        std::vector<float> out((size_t)Ta * Ha), ref(out.size()), q(Ta * nq), qr(q.size()), k(Ta * nk), kr(k.size()),
            v(Ta * nk), vr(v.size());
        attention_forward_cpu(xa.data(), aw, Ta, cfg, pos.data(), out.data(), q.data(), k.data(), v.data());
        hyo_attention_forward(xa.data(), aw.qkv_weight.data(), aw.o_weight.data(), aw.q_norm_weight.data(),
                              aw.k_norm_weight.data(), Ta, Ha, nh, nkv, hd, 1e-5f, 10000.0f, pos.data(), ref.data(),
                              qr.data(), kr.data(), vr.data());
        report(rel_err(out.data(), ref.data(), out.size()) < 1e-4 && rel_err(q.data(), qr.data(), q.size()) < 1e-4 &&
                   rel_err(k.data(), kr.data(), k.size()) < 1e-4 && rel_err(v.data(), vr.data(), v.size()) < 1e-4,
               "attention_forward_cpu (output and debug q/k/v)", errs(out.data(), ref.data(), out.size()));

        std::vector<float> rq = synth(35, 0, 0, Ta * nq, 1.0f), rk = synth(36, 0, 0, Ta * nk, 1.0f), oq = rq, ok = rk;
        rope_f32(rq.data(), rk.data(), Ta, nh, nkv, hd, 10000.0f, pos.data());
        hyo_rope_f32(oq.data(), ok.data(), Ta, nh, nkv, hd, 10000.0f, pos.data());
        report(rel_err(rq.data(), oq.data(), rq.size()) < 1e-5 && rel_err(rk.data(), ok.data(), rk.size()) < 1e-5,
               "rope_f32", errs(rq.data(), oq.data(), rq.size()));

        const uint32_t text = 3, ih = 2, iw = 3, seq = text + ih * iw;
        std::vector<float> cs(seq * hd), sn(seq * hd), csr(cs.size()), snr(sn.size());
        build_2d_rope(seq, hd, text, ih, iw, 10000.0f, cs.data(), sn.data());
        hyo_build_2d_rope(seq, hd, text, ih, iw, 10000.0f, csr.data(), snr.data());
        double dmax = 0;
        for (size_t i = 0; i < cs.size(); i++)
            dmax = std::fmax(dmax, std::fmax(std::fabs(cs[i] - csr[i]), std::fabs(sn[i] - snr[i])));
        report(dmax < 4e-6, "build_2d_rope", "max abs diff " + std::to_string(dmax));
        std::vector<float> tq = synth(37, 0, 0, seq * nq, 1.0f), tk = synth(38, 0, 0, seq * nk, 1.0f), uq = tq, uk = tk;
        apply_rope_2d_f32(tq.data(), tk.data(), csr.data(), snr.data(), seq, nh, nkv, hd);
        hyo_apply_rope_2d_f32(uq.data(), uk.data(), csr.data(), snr.data(), seq, nh, nkv, hd);
        report(rel_err(tq.data(), uq.data(), tq.size()) < 1e-6 && rel_err(tk.data(), uk.data(), tk.size()) < 1e-6,
               "apply_rope_2d_f32", errs(tq.data(), uq.data(), tq.size()));

        DecoderLayerWeights dw;
        dw.attn = aw;
        dw.input_ln_weight = synth(39, 0, 0, Ha, 0.2f);
        dw.post_attn_ln_weight = synth(40, 0, 0, Ha, 0.2f);
        for (auto& x : dw.input_ln_weight) x += 1.0f;
        for (auto& x : dw.post_attn_ln_weight) x += 1.0f;
        const uint32_t Ia = 128;
        dw.moe.num_experts = Ea;
        dw.moe.router_weight = synth(41, 1, 0, (size_t)Ea * Ha, 0.05f);
        dw.moe.shared_gate_up = synth(42, 2, Ea, (size_t)2 * Ia * Ha, 0.05f);
        dw.moe.shared_down = synth(43, 3, Ea, (size_t)Ha * Ia, 0.05f);
        dw.moe.experts.resize(Ea);
        std::vector<float> gua, dna;
        for (uint32_t e = 0; e < Ea; e++) {
            dw.moe.experts[e].gate_up = synth(44, 2, e, (size_t)2 * Ia * Ha, 0.05f);
            dw.moe.experts[e].down = synth(45, 3, e, (size_t)Ha * Ia, 0.05f);
            gua.insert(gua.end(), dw.moe.experts[e].gate_up.begin(), dw.moe.experts[e].gate_up.end());
            dna.insert(dna.end(), dw.moe.experts[e].down.begin(), dw.moe.experts[e].down.end());
        }
        cfg.num_experts = Ea;
        std::vector<float> dout((size_t)Ta * Ha), xn(dout.size()), att(dout.size()), hres(dout.size()), hn(dout.size()),
            moe(dout.size()), dref(dout.size());
        decoder_layer_forward_cpu(xa.data(), dw, Ta, cfg, pos.data(), dout.data());
        hyo_rms_norm_f32(xa.data(), dw.input_ln_weight.data(), xn.data(), Ta, Ha, 1e-5f);
        hyo_attention_forward(xn.data(), aw.qkv_weight.data(), aw.o_weight.data(), aw.q_norm_weight.data(),
                              aw.k_norm_weight.data(), Ta, Ha, nh, nkv, hd, 1e-5f, 10000.0f, pos.data(), att.data(),
                              nullptr, nullptr, nullptr);
        for (size_t i = 0; i < hres.size(); i++) hres[i] = xa[i] + att[i];
        hyo_rms_norm_f32(hres.data(), dw.post_attn_ln_weight.data(), hn.data(), Ta, Ha, 1e-5f);
        hyo_moe_forward_cpu(hn.data(), dw.moe.router_weight.data(), dw.moe.shared_gate_up.data(),
                            dw.moe.shared_down.data(), gua.data(), dna.data(), Ta, Ha, Ea, Ia, 2, moe.data(), nullptr,
                            nullptr, nullptr);
        for (size_t i = 0; i < dref.size(); i++) dref[i] = hres[i] + moe[i];
        report(rel_err(dout.data(), dref.data(), dout.size()) < 1e-4, "decoder_layer_forward_cpu",
               errs(dout.data(), dref.data(), dout.size()));

        const uint32_t Va = 40;
        std::vector<float> table = synth(46, 6, 0, (size_t)Va * Ha, 1.0f), emb((size_t)Ta * Ha);
        std::vector<int> ids(Ta);
        for (uint32_t t = 0; t < Ta; t++) ids[t] = (int)((t * 7 + 3) % Va);
        embedding_lookup_f32(ids.data(), table.data(), emb.data(), Ta, Ha);
        bool eok = true;
        for (uint32_t t = 0; t < Ta; t++) eok = eok && memcmp(&emb[(size_t)t * Ha], &table[(size_t)ids[t] * Ha], Ha * 4) == 0;
        report(eok, "embedding_lookup_f32");
        std::vector<float> lw = synth(47, 7, 0, (size_t)Va * Ha, 0.05f), lo((size_t)Ta * Va), lr(lo.size());
        lm_head_f32(xa.data(), lw.data(), lo.data(), Ta, Ha, Va);
        for (uint32_t t = 0; t < Ta; t++)
            for (uint32_t j = 0; j < Va; j++) {
                double acc = 0;
                for (uint32_t h = 0; h < Ha; h++) acc += (double)xa[(size_t)t * Ha + h] * lw[(size_t)j * Ha + h];
                lr[(size_t)t * Va + j] = (float)acc;
            }
        report(rel_err(lo.data(), lr.data(), lo.size()) < 1e-5, "lm_head_f32", errs(lo.data(), lr.data(), lo.size()));
    }
    printf("%d failure(s)\n", g_fail);
    return g_fail;
}
