// 3D RoPE tables on the host in f64 (the contract of
// ltx/block_conformance.zig:87-126): 682 frequencies theta^linspace(0,1,682)
// * pi/2 evaluated in f64 and rounded to f32 (the reference's grid generator
// returns f32), promoted back to f64 for the position products; positions
// are the (start, end) midpoints mapped to 2 * mid / max_pos - 1 with
// max_pos = (20, 2048, 2048); slot j of the 2048 per-token slots is the
// identity pad (cos 1, sin 0) for j < 2, else frequency (j - 2) / 3 on axis
// (j - 2) % 3; trig in f64, one cast to f32. Head h takes slots 64 h .. +64.
#include <cmath>
#include <thread>
#include <vector>

#include "ltx_internal.hpp"

namespace {

constexpr int kNF = 682;
constexpr double kMaxPos[3] = {20.0, 2048.0, 2048.0};

void freqs(double* f) {
    const double step = 1.0 / (double)(kNF - 1);
    for (int k = 0; k < kNF; k++) {
        const double x = k == kNF - 1 ? 1.0 : (double)k * step;  // numpy linspace
        f[k] = (double)(float)(std::pow(10000.0, x) * (M_PI / 2.0));
    }
}

}  // namespace

extern "C" int ltx_rope_tables(const float* grid, int T, float* cos_out, float* sin_out, int graph_layout) {
    try {
        if (!grid || !cos_out || !sin_out || T <= 0) throw ltx::Error("ltx_rope_tables: bad arguments");
        double f[kNF];
        freqs(f);
        auto work = [&](int t0, int t1) {
            for (int t = t0; t < t1; t++) {
                double arg[3];
                for (int a = 0; a < 3; a++) {
                    const double s0 = grid[((size_t)a * T + t) * 2], s1 = grid[((size_t)a * T + t) * 2 + 1];
                    arg[a] = (((s0 + s1) / 2.0) / kMaxPos[a]) * 2.0 - 1.0;
                }
                for (int h = 0; h < LTX_H; h++)
                    for (int k = 0; k < 64; k++) {
                        const int j = h * 64 + k;
                        double c = 1.0, s = 0.0;
                        if (j >= 2) {
                            const double th = f[(j - 2) / 3] * arg[(j - 2) % 3];
                            c = std::cos(th);
                            s = std::sin(th);
                        }
                        const size_t idx = graph_layout ? ((size_t)t * LTX_H + h) * 64 + k : ((size_t)h * T + t) * 64 + k;
                        cos_out[idx] = (float)c;
                        sin_out[idx] = (float)s;
                    }
            }
        };
        unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
        if (T < 256) nt = 1;
        std::vector<std::thread> th;
        for (unsigned i = 0; i < nt; i++) {
            int t0 = (int)((int64_t)T * i / nt), t1 = (int)((int64_t)T * (i + 1) / nt);
            th.emplace_back(work, t0, t1);
        }
        for (auto& x : th) x.join();
        return LTX_OK;
    } catch (const std::exception& ex) {
        ltx::set_thread_error(ex.what());
        return LTX_FAIL;
    }
}
