// iq_plan.h -- host-only launch planning shared by the GEMV launchers and
// the CPU tests (plain C++: no HIP types, so g++ compiles it on its own).
#pragma once

#include <algorithm>
#include <cstdint>

namespace iq {

// K ranges of a gemvq launch (M in 7..32 activation rows, G 128-column
// groups, `tiles` 16-row and `t32` 32-row tiles over all matrices, `kind`
// 0 int8 / 1 int4, `cus` compute units, `part_floats` the split-K partial
// sums the workspace holds).
//   gs  groups per range;
//   S   workgroups along K (S > 1: each writes M x tiles x 16 partial sums,
//       S of them must fit part_floats);
//   L   consecutive ranges per workgroup (1: one range each; > 1 the looped
//       kernel instance, ranges of ngl groups);
//   mb  16-row activation blocks (1 or 2).
struct GqPlan {
    int gs = 0, S = 0, L = 1, ngl = 0, mb = 0, nrb = 0;
    bool ok = false;
};

inline GqPlan gemvq_plan(int64_t G, int M, int tiles, int t32, int kind, int cus, int64_t part_floats) {
    GqPlan pl;
    if (M < 7 || M > 32 || G < 1 || tiles < 1) return pl;
    pl.nrb = (t32 + 7) / 8;
    // ranges of at most ngr groups (the weights of a range are held in
    // registers: 64 per lane at one row block; the operands of 2 blocks x 4
    // groups fill 64 KiB of LDS), and enough workgroups for two per CU
    pl.mb = M <= 16 ? 1 : 2;
    const int ngr = pl.mb == 2 ? 4 : (kind == 1 ? 6 : 4);
    const int want = 2 * cus;
    int S = int((G + ngr - 1) / ngr);
    S = std::max<int>(S, std::min<int>((want + pl.nrb - 1) / pl.nrb, int(G)));
    int gs = int((G + S - 1) / S);
    S = int((G + gs - 1) / gs);
    int L = 1;
    int ngl = ngr;
    const int64_t outs = int64_t(M) * tiles * 16;  // partial sums per workgroup along K
    if (S > 1 && int64_t(S) * outs > part_floats) {
        // partial sums beyond the workspace: fewer workgroups along K, each
        // taking L consecutive ranges; when not even two sets fit, one
        // workgroup per row block takes every range and stores y directly.
        // (int8 at two row blocks loops over 2-group ranges: 110 VGPRs,
        // two workgroups per CU, against 150 with 4)
        if (kind == 0 && pl.mb == 2) ngl = 2;
        const int R = int((G + ngl - 1) / ngl);
        gs = int((G + R - 1) / R);
        const int64_t fit = std::max<int64_t>(part_floats / outs, 1);
        L = int((R + fit - 1) / fit);
        S = (R + L - 1) / L;
    }
    pl.gs = gs;
    pl.S = S;
    pl.L = L;
    pl.ngl = ngl;
    pl.ok = S == 1 || int64_t(S) * outs <= part_floats;
    return pl;
}

}  // namespace iq
