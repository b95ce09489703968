// CPU checks of the GEMV launch plans (infer_amd/csrc/iq_plan.h): every
// plan that a launcher accepts keeps its split-K partial sums inside the
// workspace it is given and covers every 128-column group exactly once.
#include <cstdio>
#include <cstdlib>

#include "../../infer_amd/csrc/iq_plan.h"

static int failures = 0;

#define CHECK(c, ...)                         \
    do {                                      \
        if (!(c)) {                           \
            std::printf("FAIL %s: ", #c);     \
            std::printf(__VA_ARGS__);         \
            std::printf("\n");                \
            ++failures;                       \
        }                                     \
    } while (0)

int main() {
    const int64_t kStatic = int64_t(4) << 20;   // the no-allocation scratch's partial sums
    const int64_t kStream = int64_t(16) << 20;  // a per-stream workspace's
    const int64_t Ns[] = {512, 1536, 3584, 8960, 18944, 37888, 152064, 262144, 600000};
    const int64_t Ks[] = {1536, 3584, 8960, 18944};
    long plans = 0;
    for (int64_t part : {kStatic, kStream})
        for (int64_t N : Ns)
            for (int64_t K : Ks)
                for (int kind = 0; kind < 2; kind++)
                    for (int M = 7; M <= 32; M++) {
                        const int64_t G = K / 128;
                        const int tiles = int((N + 15) / 16), t32 = int((N + 31) / 32);
                        const iq::GqPlan p = iq::gemvq_plan(G, M, tiles, t32, kind, 256, part);
                        CHECK(p.ok, "N=%lld K=%lld M=%d kind=%d", (long long)N, (long long)K, M, kind);
                        if (!p.ok) continue;
                        ++plans;
                        const int64_t outs = int64_t(M) * tiles * 16;
                        CHECK(p.S == 1 || p.S * outs <= part, "partials %lld > %lld (N=%lld K=%lld M=%d kind=%d)",
                              (long long)(p.S * outs), (long long)part, (long long)N, (long long)K, M, kind);
                        // ranges r = 0 .. S*L-1 of gs groups: together they cover G, and no
                        // workgroup starts past the end
                        CHECK(int64_t(p.S) * p.L * p.gs >= G, "coverage N=%lld K=%lld M=%d", (long long)N,
                              (long long)K, M);
                        CHECK(int64_t(p.S - 1) * p.L * p.gs < G, "empty workgroup N=%lld K=%lld M=%d", (long long)N,
                              (long long)K, M);
                        CHECK(p.L == 1 || p.gs <= p.ngl, "looped range of %d groups > %d", p.gs, p.ngl);
                        CHECK(p.L > 1 || p.gs <= (p.mb == 2 ? 4 : (kind == 1 ? 6 : 4)), "range of %d groups", p.gs);
                    }
    // the case that once overflowed the static scratch: the 7B lm_head at 28..32 rows
    for (int M = 28; M <= 32; M++) {
        const iq::GqPlan p = iq::gemvq_plan(28, M, 9504, 4752, 0, 256, kStatic);
        CHECK(p.ok && p.S == 1, "lm_head M=%d S=%d", M, p.S);
    }
    std::printf("%ld plans checked, %d failures\n", plans, failures);
    return failures ? 1 : 0;
}
