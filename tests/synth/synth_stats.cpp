// Regenerates the inputs of the reference's dot-product-scaling experiment
// and prints the oracle's error statistics in the experiment's format, so
// that tests can compare them with the rows the reference committed
// (experiments/dot-product-scaling/results/{synth,convert}.jsonl).
//
// TEST INFRASTRUCTURE ONLY: links the CPU oracle (oracle/lns_oracle.c).
//
// The experiment's generator is std::mt19937_64 seeded with seed + K and
// std::normal_distribution<float>(0, 1) (dot-bench.cpp:103-131, :134-140),
// built with g++ (experiments/dot-product-scaling/run.py:31-38), so the same
// libstdc++ calls here give the same operands.  Outputs per K: 4096, N = 4
// activation rows, M = 1024 weight rows; the statistics are those of
// dot-bench.cpp:82-101 over the "acc" error (got - exact) / sum|products|,
// exact being the long-double dot of the LNS-rounded operands.
//
// usage: synth_stats synth <base|monte|lpvip|sum32|xlns32> <signed|positive|attn> <kmin> <kmax> [xlns32 variant]
//        synth_stats convert <xlns16|xlns32>
//        synth_stats monte <signed|positive|attn> <kmin> <kmax> <reps> <outputs>
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "lns_oracle.h"

namespace {

struct Stats {
    double n = 0, sum = 0, sumsq = 0, abs_sum = 0, num = 0, den = 0;
    void add(long double got, long double ref, long double scale) {
        const double e = scale > 0 ? (double)((got - ref) / scale) : 0.0;
        n += 1;
        sum += e;
        sumsq += e * e;
        abs_sum += std::fabs(e);
        num += (double)((got - ref) * (got - ref));
        den += (double)(ref * ref);
    }
    void print(const char *cfg, const char *dist, long long K) const {
        const double mean = sum / n;
        std::printf("{\"config\":\"%s\",\"dist\":\"%s\",\"K\":%lld,\"acc\":{\"bias\":%.6g,\"sd\":%.6g,\"rms\":%.6g,"
                    "\"mean_abs\":%.6g,\"rel_l2\":%.6g}}\n",
                    cfg, dist, K, mean, std::sqrt(std::max(0.0, sumsq / n - mean * mean)), std::sqrt(sumsq / n),
                    abs_sum / n, den > 0 ? std::sqrt(num / den) : 0.0);
    }
};

// operands of one K (dot-bench.cpp's gen_inputs: a first, then x)
void operands(const std::string &dist, int64_t K, int64_t M, int64_t N, std::mt19937_64 &rng,
              std::vector<float> &a, std::vector<float> &x) {
    std::normal_distribution<float> g(0.0f, 1.0f);
    a.resize((size_t)(K * M));
    x.resize((size_t)(K * N));
    for (float &v : a) v = g(rng);
    if (dist == "signed") {
        for (float &v : x) v = g(rng);
    } else if (dist == "positive") {
        for (float &v : a) v = std::fabs(v);
        for (float &v : x) v = std::fabs(g(rng));
    } else {   // attn: softmax rows of 2 N(0,1) logits
        for (int64_t n = 0; n < N; n++) {
            float *r = &x[(size_t)(n * K)];
            float mx = -1e30f;
            for (int64_t k = 0; k < K; k++) {
                r[k] = 2.0f * g(rng);
                mx = std::max(mx, r[k]);
            }
            double s = 0;
            for (int64_t k = 0; k < K; k++) {
                r[k] = std::exp(r[k] - mx);
                s += r[k];
            }
            for (int64_t k = 0; k < K; k++) r[k] = (float)(r[k] / s);
        }
    }
}

void round16(const std::vector<float> &v, std::vector<float> &out) {
    out.resize(v.size());
    for (size_t i = 0; i < v.size(); i++) out[i] = lno16_to_f32(lno16_from_f32(v[i]));
}

void round32(const std::vector<float> &v, std::vector<float> &out) {
    out.resize(v.size());
    for (size_t i = 0; i < v.size(); i++) out[i] = lno32_to_f32(lno32_from_f32(v[i]));
}

int synth(const std::string &cfg, const std::string &dist, int64_t kmin, int64_t kmax) {
    const uint64_t seed = 1;
    const int64_t N = 4, M = 1024;
    const bool x32 = cfg == "xlns32";
    int mode = LNO_BASE;
    if (cfg == "monte") mode = LNO_MONTE;
    else if (cfg == "lpvip") mode = LNO_LPVIP;
    else if (cfg == "sum32") mode = LNO_SUM32;
    else if (cfg != "base" && !x32) return 2;
    for (int64_t K = kmin; K <= kmax; K *= 2) {
        std::mt19937_64 rng(seed + (uint64_t)K);
        std::vector<float> a0, x0, a, x;
        operands(dist, K, M, N, rng, a0, x0);
        if (x32) {
            round32(a0, a);
            round32(x0, x);
        } else {
            round16(a0, a);
            round16(x0, x);
        }
        // Monte: the experiment sets the LFSR before each product (dot-bench.cpp:148)
        if (mode == LNO_MONTE) lno_monte_set_state((uint16_t)(1 + (seed * 7919 + (uint64_t)K) % 65535));
        std::vector<float> out((size_t)(M * N));
        if (x32) lno32_mul_mat(a0.data(), x0.data(), out.data(), K, M, N, 1, 1, 1, 1);
        else lno16_mul_mat_f32w(mode, a0.data(), x0.data(), out.data(), K, M, N, 1, 1, 1, 1);
        Stats st;
        for (int64_t n = 0; n < N; n++) {
            for (int64_t m = 0; m < M; m++) {
                long double s = 0, s1 = 0;
                for (int64_t k = 0; k < K; k++) {
                    const long double p = (long double)a[(size_t)(m * K + k)] * (long double)x[(size_t)(n * K + k)];
                    s += p;
                    s1 += fabsl(p);
                }
                st.add(out[(size_t)(n * M + m)], s, s1);
            }
        }
        st.print(cfg.c_str(), dist.c_str(), (long long)K);
        std::fflush(stdout);
    }
    return 0;
}

// The experiment's Monte rows (results/monte.jsonl, run.py:98-105:
// dot-bench.cpp synth with --reps 32 --outputs 2048): M = outputs / 4, the
// LFSR set before each rep's product from (seed, rep, K)
// (dot-bench.cpp:149-150), rep 0's "acc" statistics, then those of the mean
// over the first 1, 2, 4, ... reps of every output (dot-bench.cpp:166-177).
int monte_reps(const std::string &dist, int64_t kmin, int64_t kmax, int reps, int64_t outputs) {
    const uint64_t seed = 1;
    const int64_t N = 4, M = std::max<int64_t>(1, outputs / N);
    for (int64_t K = kmin; K <= kmax; K *= 2) {
        std::mt19937_64 rng(seed + (uint64_t)K);
        std::vector<float> a0, x0, a, x;
        operands(dist, K, M, N, rng, a0, x0);
        round16(a0, a);
        round16(x0, x);
        std::vector<long double> s((size_t)(M * N)), s1((size_t)(M * N));
        for (int64_t n = 0; n < N; n++)
            for (int64_t m = 0; m < M; m++) {
                long double t = 0, t1 = 0;
                for (int64_t k = 0; k < K; k++) {
                    const long double p = (long double)a[(size_t)(m * K + k)] * (long double)x[(size_t)(n * K + k)];
                    t += p;
                    t1 += fabsl(p);
                }
                s[(size_t)(n * M + m)] = t;
                s1[(size_t)(n * M + m)] = t1;
            }
        std::vector<std::vector<float>> outs((size_t)reps, std::vector<float>((size_t)(M * N)));
        for (int r = 0; r < reps; r++) {
            lno_monte_set_state((uint16_t)(1 + (seed * 7919 + (uint64_t)r * 104729 + (uint64_t)K) % 65535));
            lno16_mul_mat_f32w(LNO_MONTE, a0.data(), x0.data(), outs[(size_t)r].data(), K, M, N, 1, 1, 1, 1);
        }
        Stats st;
        for (size_t i = 0; i < s.size(); i++) st.add(outs[0][i], s[i], s1[i]);
        st.print("monte", dist.c_str(), (long long)K);
        for (int r = 1; r <= reps; r *= 2) {
            Stats sa;
            for (size_t i = 0; i < s.size(); i++) {
                long double m = 0;
                for (int q = 0; q < r; q++) m += outs[(size_t)q][i];
                sa.add(m / r, s[i], s1[i]);
            }
            const double mean = sa.sum / sa.n;
            std::printf("{\"avg\":{\"dist\":\"%s\",\"K\":%lld,\"reps\":%d,\"bias\":%.6g,\"sd\":%.6g,\"rms\":%.6g}}\n",
                        dist.c_str(), (long long)K, r, mean, std::sqrt(std::max(0.0, sa.sumsq / sa.n - mean * mean)),
                        std::sqrt(sa.sumsq / sa.n));
        }
        std::fflush(stdout);
    }
    return 0;
}

// dot-bench.cpp:186-218: 4M log-uniform values, three round trips
int convert(const std::string &fmt) {
    const bool x32 = fmt == "xlns32";
    std::mt19937_64 rng(1);
    std::uniform_real_distribution<double> e(-20.0, 20.0);
    std::vector<float> v((size_t)4194304), r1, r2, r3;
    for (float &x : v) {
        const double s = (rng() & 1) ? -1.0 : 1.0;
        x = (float)(s * std::exp2(e(rng)));
    }
    auto rt = x32 ? round32 : round16;
    rt(v, r1);
    rt(r1, r2);
    rt(r2, r3);
    double mean = 0, sq = 0, lg = 0, d12 = 0, d23 = 0;
    long long up = 0, down = 0, same = 0, ch12 = 0, ch23 = 0, cnt = 0;
    for (size_t i = 0; i < v.size(); i++) {
        if (!std::isfinite(r1[i]) || !std::isfinite(r3[i]) || r1[i] == 0 || r2[i] == 0 || r3[i] == 0) continue;
        const double rel = ((double)r1[i] - v[i]) / v[i];
        mean += rel;
        sq += rel * rel;
        lg += std::log2(std::fabs((double)r1[i] / v[i]));
        up += std::fabs(r1[i]) > std::fabs(v[i]);
        down += std::fabs(r1[i]) < std::fabs(v[i]);
        same += r1[i] == v[i];
        ch12 += r2[i] != r1[i];
        ch23 += r3[i] != r2[i];
        d12 += std::log2(std::fabs((double)r2[i] / r1[i]));
        d23 += std::log2(std::fabs((double)r3[i] / r2[i]));
        cnt++;
    }
    const double c = (double)cnt;
    std::printf("{\"values\":%lld,\"mean_rel\":%.6g,\"rms_rel\":%.6g,\"mean_log2\":%.6g,\"frac_up\":%.6g,"
                "\"frac_down\":%.6g,\"frac_exact\":%.6g,\"frac_changed_round2\":%.6g,\"frac_changed_round3\":%.6g,"
                "\"drift_log2_round2\":%.6g,\"drift_log2_round3\":%.6g}\n",
                cnt, mean / c, std::sqrt(sq / c), lg / c, up / c, down / c, same / c, ch12 / c, ch23 / c, d12 / c,
                d23 / c);
    return 0;
}

}  // namespace

int main(int argc, char **argv) {
    lno_init();
    if (argc >= 6 && !std::strcmp(argv[1], "synth")) {
        if (argc >= 7) lno32_set_variant(std::atoi(argv[6]));
        return synth(argv[2], argv[3], std::atoll(argv[4]), std::atoll(argv[5]));
    }
    if (argc >= 3 && !std::strcmp(argv[1], "convert")) return convert(argv[2]);
    if (argc >= 7 && !std::strcmp(argv[1], "monte"))
        return monte_reps(argv[2], std::atoll(argv[3]), std::atoll(argv[4]), std::atoi(argv[5]), std::atoll(argv[6]));
    std::fprintf(stderr, "usage: %s synth CFG DIST KMIN KMAX [VARIANT] | convert FMT | monte DIST KMIN KMAX REPS OUTPUTS\n",
                 argv[0]);
    return 2;
}
