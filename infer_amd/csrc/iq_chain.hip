// iq_chain.hip -- a chain of dependent 1-row quantised GEMVs in one
// persistent launch: the quantised part of the reference's decode step
// (GpuBatch::Impl::launch_sequence, kernels/batch_gpu.cu:186-215) as a
// program of stages, each stage one linear call site (q|k|v, o, gate|up
// with the SwiGLU of kernels/ops/elementwise.cu:6-11 as its epilogue, down,
// the LM head) whose input is the output of an earlier stage.
//
// Why one launch: a decode-step GEMV streams 7-70 MB and is over in 4-16 us,
// of which 3-5 us per launch are ramp-up, the first-load latency and the
// tail of the last workgroups.  Here one workgroup per CU stays resident for
// the whole program; between dependent stages it crosses a grid barrier, and
// because the weights of a GEMV do not depend on its input, each workgroup
// requests the weights of its first slices of stage s+1 before it waits for
// the other workgroups to finish stage s.  The HBM stream continues across
// the barrier instead of draining and refilling at every kernel boundary.
//
// Arithmetic per slice is the 1-row GEMV's (iq_limbs.h): the stage input is
// converted once per workgroup into byte limbs in LDS, codes x limbs on
// v_mfma_i32_16x16x64_i8 give exact int32 sums, combine() applies scale,
// zero point and the activation exponent in fp32.
//
// Work split.  A stage's work units are 16-row output tiles (or, for the
// SwiGLU epilogue, a gate tile with the up tile of the same rows); unit u
// belongs to workgroup u mod W.  A unit's K range is cut into slices of
// kSliceGroups 128-column groups; the 16 waves of a workgroup take 16
// consecutive slices of the workgroup's list at a time, each holding the
// next slice's weights in registers while it multiplies the current one.
// Slice sums go to LDS and are added per tile in slice order (deterministic)
// when the stage's slices are done.
//
// Coherence without cache maintenance.  The L2 is per XCD and not coherent
// across XCDs, so: (1) every stage output is stored with agent-scope
// (write-through) stores and waited for before the workgroup arrives at the
// barrier; (2) every vector a stage reads was written by an earlier stage of
// the same launch and is never written again in it (the host checks this
// single-assignment rule), so no XCD can hold a stale copy of a line it
// reads: the launch starts with invalidated L2s, and each line is first
// touched after its producer's stores reached memory.
//
// Grid barrier: one counter, incremented once per workgroup and stage,
// polled by one thread per workgroup; the launch is cooperative (every
// workgroup resident), and the poll gives up after a bounded number of
// sleeps (flag set, kernel exits normally) so that a broken launch cannot
// hang the device.
#include <algorithm>
#include <cstring>
#include <mutex>
#include <vector>

#include "../../include/iq.h"
#include "iq_limbs.h"

namespace iq {

namespace {

constexpr int kWaves = 16;         // waves per workgroup
// A wave slice is 64 bytes of codes per lane: 4 groups of int4 or 2 of int8.
constexpr int kSliceDw = 4;        // 16-byte weight registers per slice
constexpr int kMaxPasses = 3;      // conversion passes (64 groups each): K <= 24576
constexpr int kMaxStageMats = 3;

struct CMat {
    const uint8_t* q;
    const uint16_t* scales;
    const uint8_t* zeros;
    const uint16_t* bias;
    float* y;
    int32_t N;
    int32_t tile0;  // first tile of this matrix in the stage's tile numbering
};

struct CStage {
    CMat mat[kMaxStageMats];
    const float* x;
    const uint16_t* norm;
    const float* res;
    float eps;
    int32_t kind, in_op, out_op, nmat;
    int32_t K, G;
    int32_t units;   // work units
    int32_t tpu;     // tiles per unit (2: SwiGLU pair)
    int32_t chunks;  // slices per tile
    int32_t gsl;     // groups per slice (4 int4, 2 int8)
    int32_t gqa_hd, gqa_span;  // IQ_IN_GQA: head_dim, head_dim * group
};

struct CParams {
    const CStage* st;
    int nst;
    int* bar;        // [0] arrival counter, [1] timeout flag
    int spin_limit;  // sleeps before a barrier wait gives up
};

// Weights, scales and zero points of one wave slice.
// int4: w[g] = the lane's 16 bytes of group g < 4; int8: w[2g], w[2g + 1]
// for g < 2.
struct SliceRegs {
    int4v_t w[kSliceDw];
    uint32_t s[2];  // bf16 scales, groups (0,1) and (2,3)
    uint32_t z;     // int4 zero points, one byte per group
};

// The slice a wave handles: tile, K groups [g0, g0 + gs), LDS slot.
struct SliceRef {
    int valid;
    int slot;   // index into the workgroup's slice sums
    int mat;
    int64_t row0;
    int g0, gs;
};

__device__ __forceinline__ int units_of(const CStage& st, int wg, int W) {
    return st.units > wg ? (st.units - wg + W - 1) / W : 0;
}

__device__ __forceinline__ SliceRef slice_ref(const CStage& st, int wg, int W, int idx) {
    SliceRef r{0, idx, 0, 0, 0, 0};
    const int per_unit = st.tpu * st.chunks;
    const int nsl = units_of(st, wg, W) * per_unit;
    if (idx >= nsl) return r;
    const int j = idx / per_unit, rem = idx - j * per_unit;
    const int p = rem / st.chunks, c = rem - p * st.chunks;
    const int u = wg + j * W;
    int m = 0, tile;
    if (st.tpu == 2) {
        m = p;
        tile = u;  // tile u of gate (p = 0) and of up (p = 1)
    } else {
        tile = u;
        for (int i = 1; i < kMaxStageMats; i++)
            if (i < st.nmat && tile >= st.mat[i].tile0) m = i;
        tile -= st.mat[m].tile0;
    }
    r.valid = 1;
    r.mat = m;
    r.row0 = int64_t(tile) * 16;
    r.g0 = c * st.gsl;
    r.gs = st.G - r.g0 < st.gsl ? st.G - r.g0 : st.gsl;
    return r;
}

// Requests one slice's weights, scales and zero points (rows past N and
// groups past the slice read zero without a memory access).
__device__ __forceinline__ void load_slice(SliceRegs& b, const CStage& st, const SliceRef& r, int ln, int kg) {
    const CMat& m = st.mat[r.mat];
    const int64_t row = r.row0 + ln;
    const int G = st.G;
    const int kind = st.kind;
    const int64_t rb = kind == 1 ? st.K / 2 : st.K;
    const rsrc_t rq = make_rsrc(m.q, r.valid ? int64_t(m.N) * rb : 0);
    const rsrc_t rs = make_rsrc(m.scales, r.valid ? int64_t(m.N) * G * 2 : 0);
    const rsrc_t rz = make_rsrc(m.zeros, (r.valid && kind == 1) ? int64_t(m.N) * G : 0);
    const uint32_t vq = uint32_t(row * rb) + uint32_t(r.g0 * (kind == 1 ? 64 : 128) + kg * 16);
    if (kind == 1) {
#pragma unroll
        for (int gl = 0; gl < 4; gl++)
            b.w[gl] = __builtin_bit_cast(
                int4v_t, __builtin_amdgcn_raw_buffer_load_b128(rq, vq + (gl < r.gs ? 0u : kOob), gl * 64, 0));
    } else {
#pragma unroll
        for (int gl = 0; gl < 2; gl++)
#pragma unroll
            for (int h = 0; h < 2; h++)
                b.w[2 * gl + h] = __builtin_bit_cast(
                    int4v_t, __builtin_amdgcn_raw_buffer_load_b128(rq, vq + (gl < r.gs ? 0u : kOob), gl * 128 + h * 64, 0));
    }
    // G is even and g0 even: scales of groups (2i, 2i + 1) are one 4-byte
    // word, their zero points one 2-byte word
    const uint32_t vs = uint32_t((row * G + r.g0) * 2), vz = uint32_t(row * G + r.g0);
#pragma unroll
    for (int i = 0; i < 2; i++) b.s[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, vs + (2 * i < r.gs ? 0u : kOob), 4 * i, 0);
    if (kind == 1) {
        const uint32_t z0 = __builtin_amdgcn_raw_buffer_load_b16(rz, vz, 0, 0);
        const uint32_t z1 = __builtin_amdgcn_raw_buffer_load_b16(rz, vz + (2 < r.gs ? 0u : kOob), 2, 0);
        b.z = z0 | (z1 << 16);
    } else {
        b.z = 0;
    }
}

// Sum over the slice of codes x converted activations for the lane's row
// (lanes 0..15 hold rows row0 + ln; other lanes' values are unused).
__device__ __forceinline__ float slice_sum(const SliceRegs& b, const SliceRef& r, int kind, const int8_t* xs,
                                           const int4* ms, int ln, int kg) {
    float acc = 0.0f;
    const bool alive = ln < 3;  // A rows 0..2 carry limbs 0..2
#pragma unroll
    for (int gl = 0; gl < 4; gl++) {
        if (kind != 1 && gl >= 2) break;
        if (gl >= r.gs) break;  // wave-uniform
        const int g = r.g0 + gl;
        int4v_t a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0};
        if (alive) {
            const int8_t* pa = xs + g * kLimbRec + ln * kGroup + kg * 16;
            a0 = *reinterpret_cast<const int4v_t*>(pa);
            a1 = *reinterpret_cast<const int4v_t*>(pa + 64);
        }
        int4v_t b0, b1;
        if (kind == 1) {
            const int4v_t v = b.w[gl];
            b0 = v & 0x0F0F0F0F;
            b1 = (v >> 4) & 0x0F0F0F0F;
        } else {
            b0 = b.w[(2 * gl) & 3];
            b1 = b.w[(2 * gl + 1) & 3];
        }
        int4v_t D = mfma_i8(a0, b0, int4v_t{0, 0, 0, 0});
        D = mfma_i8(a1, b1, D);
        const uint32_t sw = b.s[gl >> 1];
        const float sc = __uint_as_float((gl & 1) ? (sw & 0xFFFF0000u) : (sw << 16));
        const int z = kind == 1 ? int((b.z >> (8 * gl)) & 0xFF) : 0;
        acc = combine(acc, D[0], D[1], D[2], z, ms[g], sc);
    }
    return acc;
}

// Columns [k0, k0 + 8) of the stage input, before normalisation.
__device__ __forceinline__ void load_input8(const CStage& st, int k0, float (&v)[8]) {
    const float* src = st.x + k0;
    if (st.in_op == IQ_IN_GQA) {
        // query-head column k0 reads the value row of its key/value head
        const int span = st.gqa_span, hd = st.gqa_hd;
        src = st.x + (k0 / span) * hd + (k0 % hd);
    }
    const float4 a = *reinterpret_cast<const float4*>(src);
    const float4 c = *reinterpret_cast<const float4*>(src + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = c.x; v[5] = c.y; v[6] = c.z; v[7] = c.w;
}

// Full-wave sum of a double, every lane gets the total (fixed order).
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__global__ __launch_bounds__(64 * kWaves) void chain_kernel(const CParams P) {
    extern __shared__ __attribute__((aligned(16))) int8_t lds[];
    __shared__ double ssq[kWaves];
    const int tid = threadIdx.x, lane = tid & 63, ln = lane & 15, kg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wg = blockIdx.x, W = gridDim.x;
    // LDS: limb records [G][384] | meta [G] int4 | slice sums [slots][16]
    int8_t* xs = lds;

    SliceRegs B0, B1;
    {
        const CStage& st = P.st[0];
        load_slice(B0, st, slice_ref(st, wg, W, wave), ln, kg);
    }
    for (int s = 0; s < P.nst; s++) {
        const CStage& st = P.st[s];
        const int G = st.G;
        int4* ms = reinterpret_cast<int4*>(lds + G * kLimbRec);
        float* red = reinterpret_cast<float*>(lds + G * (kLimbRec + 16));
        if (s > 0) {
            // every workgroup has stored its outputs of stages < s
            if (tid == 0) {
                const int target = W * s;
                int n = 0;
                while (__hip_atomic_load(P.bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
                    if (++n > P.spin_limit) {
                        __hip_atomic_store(P.bar + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                }
            }
            __syncthreads();
        }

        // 1. The stage input into limb records: pass t, wave w, lane row kg
        //    converts group 64 t + 4 w + kg (16 lanes x 8 columns).
        {
            const bool perm = st.kind == 1;
            float v[kMaxPasses][8];
            double part = 0.0;
#pragma unroll
            for (int t = 0; t < kMaxPasses; t++) {
                const int g = 64 * t + 4 * wave + kg;
#pragma unroll
                for (int i = 0; i < 8; i++) v[t][i] = 0.0f;
                if (64 * t + 4 * wave < G) {  // wave-uniform
                    if (g < G) load_input8(st, g * kGroup + ln * 8, v[t]);
#pragma unroll
                    for (int i = 0; i < 8; i++) part += double(v[t][i]) * double(v[t][i]);
                }
            }
            if (st.in_op == IQ_IN_RMSNORM) {
                // x / sqrt(mean(x^2) + eps) * w   (src/forward.cpp:21-31)
                part = wave_sum(part);
                if (lane == 0) ssq[wave] = part;
                __syncthreads();
                double ss = 0.0;
#pragma unroll
                for (int w = 0; w < kWaves; w++) ss += ssq[w];
                const float scale = 1.0f / __builtin_sqrtf(float(ss / double(st.K)) + st.eps);
#pragma unroll
                for (int t = 0; t < kMaxPasses; t++) {
                    const int g = 64 * t + 4 * wave + kg;
                    if (64 * t + 4 * wave < G && g < G) {
                        const uint4 nb = *reinterpret_cast<const uint4*>(st.norm + g * kGroup + ln * 8);
                        const uint32_t nw[4] = {nb.x, nb.y, nb.z, nb.w};
#pragma unroll
                        for (int i = 0; i < 8; i++) {
                            const float w = __uint_as_float((i & 1) ? (nw[i >> 1] & 0xFFFF0000u) : (nw[i >> 1] << 16));
                            v[t][i] = (v[t][i] * scale) * w;
                        }
                    }
                }
            }
#pragma unroll
            for (int t = 0; t < kMaxPasses; t++) {
                const int g = 64 * t + 4 * wave + kg;
                if (64 * t + 4 * wave >= G) break;  // wave-uniform
                const bool ok = g < G;
                int4 md;
                if (perm) md = convert_group<true>(v[t], ln, ok, xs + (ok ? g : 0) * kLimbRec);
                else md = convert_group<false>(v[t], ln, ok, xs + (ok ? g : 0) * kLimbRec);
                if (ok && ln == 0) ms[g] = md;
            }
        }
        __syncthreads();

        // 2. This workgroup's slices, 16 at a time, the next one's weights
        //    in flight while the current one is multiplied.
        const int nsl = units_of(st, wg, W) * st.tpu * st.chunks;
        const int nit = (nsl + kWaves - 1) / kWaves;
        for (int it = 0; it < nit; it += 2) {
            const SliceRef r0 = slice_ref(st, wg, W, it * kWaves + wave);
            const SliceRef r1 = slice_ref(st, wg, W, (it + 1) * kWaves + wave);
            if (it + 1 < nit) load_slice(B1, st, r1, ln, kg);
            if (r0.valid) {
                const float a = slice_sum(B0, r0, st.kind, xs, ms, ln, kg);
                if (lane < 16) red[r0.slot * 16 + ln] = a;
            }
            if (it + 1 >= nit) break;
            if (it + 2 < nit) load_slice(B0, st, slice_ref(st, wg, W, (it + 2) * kWaves + wave), ln, kg);
            if (r1.valid) {
                const float a = slice_sum(B1, r1, st.kind, xs, ms, ln, kg);
                if (lane < 16) red[r1.slot * 16 + ln] = a;
            }
        }
        __syncthreads();

        // 3. Per unit: slice sums in slice order, the epilogue, write-through
        //    stores (wave j % 16 finalises unit j, lanes 0..15 its rows).
        const int nu = units_of(st, wg, W);
        for (int j = wave; j < nu; j += kWaves) {
            if (lane >= 16) continue;
            const int u = wg + j * W;
            float acc[2] = {0.0f, 0.0f};
#pragma unroll
            for (int p = 0; p < 2; p++) {
                if (p >= st.tpu) break;
                const float* rp = red + ((j * st.tpu + p) * st.chunks) * 16 + ln;
                float sum = 0.0f;
                for (int c = 0; c < st.chunks; c++) sum += rp[c * 16];
                acc[p] = sum;
            }
            int m = 0, tile = u;
            if (st.tpu == 1) {
                for (int i = 1; i < kMaxStageMats; i++)
                    if (i < st.nmat && u >= st.mat[i].tile0) m = i;
                tile = u - st.mat[m].tile0;
            }
            const CMat& M = st.mat[m];
            const int64_t row = int64_t(tile) * 16 + ln;
            if (row >= M.N) continue;
            float out;
            if (st.out_op == IQ_OUT_SWIGLU) {
                // silu(g) * u  (kernels/ops/elementwise.cu:6-11)
                const float g = acc[0] + (st.mat[0].bias ? bf16_to_f32(st.mat[0].bias[row]) : 0.0f);
                const float up = acc[1] + (st.mat[1].bias ? bf16_to_f32(st.mat[1].bias[row]) : 0.0f);
                out = g / (1.0f + expf(-g)) * up;
            } else {
                out = acc[0] + (M.bias ? bf16_to_f32(M.bias[row]) : 0.0f);
                if (st.out_op == IQ_OUT_RESIDUAL) out = st.res[row] + out;
            }
            __hip_atomic_store(M.y + row, out, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // stores complete (written through) before this workgroup arrives;
        // only then the next stage's first weights are requested
        __builtin_amdgcn_s_waitcnt(0);
        if (s + 1 < P.nst) {
            const CStage& nx = P.st[s + 1];
            load_slice(B0, nx, slice_ref(nx, wg, W, wave), ln, kg);
        }
        __syncthreads();
        if (tid == 0 && s + 1 < P.nst) __hip_atomic_fetch_add(P.bar, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

__global__ void chain_reset_kernel(int* bar) {
    if (threadIdx.x < 2) bar[threadIdx.x] = 0;
}

}  // namespace

// Host side of a chain: the validated program on the device.
struct Chain {
    int device = 0;
    int nst = 0;
    int W = 0;
    size_t lds = 0;
    CStage* d_st = nullptr;
    int* d_bar = nullptr;
};

namespace {

struct Range {
    uintptr_t lo, hi;
};
bool overlaps(const Range& a, const Range& b) { return a.lo < b.hi && b.lo < a.hi; }

}  // namespace

int chain_create(const iq_stage* stages, int n, Chain** out) {
    if (!stages || !out) return IQ_ENULL;
    *out = nullptr;
    if (n < 1) return IQ_ESHAPE;
    std::vector<CStage> prog(static_cast<size_t>(n));
    std::vector<std::vector<Range>> reads(static_cast<size_t>(n)), writes(static_cast<size_t>(n));
    size_t lds_max = 0;
    const int cus = device_cu_count();
    for (int s = 0; s < n; s++) {
        const iq_stage& a = stages[s];
        CStage& c = prog[size_t(s)];
        std::memset(&c, 0, sizeof(c));
        if (a.n < 1 || a.n > kMaxStageMats) return IQ_ESHAPE;
        if (a.in_op < IQ_IN_PLAIN || a.in_op > IQ_IN_GQA) return IQ_ESHAPE;
        if (a.out_op < IQ_OUT_STORE || a.out_op > IQ_OUT_SWIGLU) return IQ_ESHAPE;
        const iq_view& W0 = a.W[0];
        if (W0.kind != IQ_INT8 && W0.kind != IQ_INT4) return IQ_EKIND;
        const int64_t K = W0.cols, G = (K + kGroup - 1) / kGroup;
        // whole groups, an even group count (paired scale loads), at most
        // three conversion passes
        if (K <= 0 || K % (2 * kGroup) || G > 64 * kMaxPasses) return IQ_ESHAPE;
        int tiles = 0;
        for (int i = 0; i < a.n; i++) {
            const iq_view& Wi = a.W[i];
            if (Wi.kind != W0.kind) return IQ_EKIND;
            if (Wi.cols != K || Wi.groups != G || Wi.rows <= 0 || Wi.rows > (int64_t(1) << 30)) return IQ_ESHAPE;
            if (!Wi.q || !Wi.scales || (Wi.kind == IQ_INT4 && !Wi.zeros)) return IQ_ENULL;
            const int64_t rb = Wi.kind == IQ_INT4 ? K / 2 : K;
            if (Wi.rows * rb >= (int64_t(1) << 31)) return IQ_ETOOLARGE;
            c.mat[i] = CMat{Wi.q, Wi.scales, Wi.kind == IQ_INT4 ? Wi.zeros : nullptr, a.bias[i], a.y[i],
                            int32_t(Wi.rows), tiles};
            tiles += int((Wi.rows + 15) / 16);
        }
        const bool pair = a.out_op == IQ_OUT_SWIGLU;
        if (pair && (a.n != 2 || a.W[1].rows != W0.rows)) return IQ_ESHAPE;
        const int nout = pair ? 1 : a.n;
        for (int i = 0; i < nout; i++) {
            if (!a.y[i]) return IQ_ENULL;
            if (reinterpret_cast<uintptr_t>(a.y[i]) % 4) return IQ_ESHAPE;
            writes[size_t(s)].push_back({reinterpret_cast<uintptr_t>(a.y[i]),
                                         reinterpret_cast<uintptr_t>(a.y[i] + a.W[i].rows)});
        }
        if (!a.x) return IQ_ENULL;
        if (reinterpret_cast<uintptr_t>(a.x) % 16) return IQ_ESHAPE;
        int64_t xlen = K;
        if (a.in_op == IQ_IN_GQA) {
            const int64_t hd = a.gqa_head_dim, grp = a.gqa_group;
            if (hd <= 0 || hd % 8 || grp <= 0 || K % (hd * grp)) return IQ_ESHAPE;
            c.gqa_hd = int32_t(hd);
            c.gqa_span = int32_t(hd * grp);
            xlen = K / grp;
        }
        reads[size_t(s)].push_back({reinterpret_cast<uintptr_t>(a.x), reinterpret_cast<uintptr_t>(a.x + xlen)});
        if (a.in_op == IQ_IN_RMSNORM) {
            if (!a.norm) return IQ_ENULL;
            if (reinterpret_cast<uintptr_t>(a.norm) % 16) return IQ_ESHAPE;
            if (!(a.eps >= 0.0f)) return IQ_ESHAPE;
        }
        if (a.out_op == IQ_OUT_RESIDUAL) {
            if (!a.residual) return IQ_ENULL;
            reads[size_t(s)].push_back({reinterpret_cast<uintptr_t>(a.residual),
                                        reinterpret_cast<uintptr_t>(a.residual + W0.rows)});
            if (a.n != 1) return IQ_ESHAPE;
        }
        c.x = a.x;
        c.norm = a.norm;
        c.res = a.residual;
        c.eps = a.eps;
        c.kind = W0.kind;
        c.in_op = a.in_op;
        c.out_op = a.out_op;
        c.nmat = a.n;
        c.K = int32_t(K);
        c.G = int32_t(G);
        c.tpu = pair ? 2 : 1;
        c.units = pair ? int((W0.rows + 15) / 16) : tiles;
        c.gsl = W0.kind == IQ_INT4 ? 4 : 2;
        c.chunks = int((G + c.gsl - 1) / c.gsl);
        const int64_t per_wg = (c.units + cus - 1) / cus;
        const size_t lds = size_t(G) * (kLimbRec + 16) + size_t(per_wg) * c.tpu * c.chunks * 16 * sizeof(float);
        lds_max = std::max(lds_max, lds);
    }
    // Single assignment: a stage writes nothing that it or an earlier stage
    // reads or writes (a rewritten line could be stale in another XCD's L2).
    for (int s = 0; s < n; s++)
        for (const Range& w : writes[size_t(s)])
            for (int e = 0; e <= s; e++) {
                for (const Range& r : reads[size_t(e)])
                    if (overlaps(w, r)) return IQ_EALIAS;
                for (const Range& o : writes[size_t(e)])
                    if ((e < s || &o != &w) && overlaps(w, o)) return IQ_EALIAS;
            }
    if (lds_max > 160 * 1024) return IQ_ETOOLARGE;

    Chain* ch = new Chain();
    hipError_t e = hipGetDevice(&ch->device);
    int occ = 0;
    if (e == hipSuccess)
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(chain_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, int(lds_max));
    if (e == hipSuccess)
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(chain_kernel), 64 * kWaves,
                                                          lds_max);
    if (e == hipSuccess && occ < 1) e = hipErrorCooperativeLaunchTooLarge;
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&ch->d_st), sizeof(CStage) * size_t(n));
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&ch->d_bar), 256);
    if (e == hipSuccess) e = hipMemcpy(ch->d_st, prog.data(), sizeof(CStage) * size_t(n), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset(ch->d_bar, 0, 256);
    if (e != hipSuccess) {
        chain_destroy(ch);
        return e == hipErrorOutOfMemory ? IQ_ENOMEM : int(e);
    }
    ch->nst = n;
    ch->W = cus;
    ch->lds = lds_max;
    *out = ch;
    return IQ_OK;
}

hipError_t chain_run(const Chain* ch, hipStream_t stream) {
    chain_reset_kernel<<<1, 64, 0, stream>>>(ch->d_bar);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    CParams p;
    p.st = ch->d_st;
    p.nst = ch->nst;
    p.bar = ch->d_bar;
    p.spin_limit = 1 << 22;  // ~0.1-0.5 s of sleeps per barrier
    void* args[] = {&p};
    return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(chain_kernel), dim3(unsigned(ch->W)),
                                      dim3(64 * kWaves), args, ch->lds, stream);
}

int chain_timed_out(const Chain* ch, int* flag) {
    int v[2] = {0, 0};
    const hipError_t e = hipMemcpy(v, ch->d_bar, sizeof(v), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return int(e);
    *flag = v[1];
    return IQ_OK;
}

void chain_destroy(Chain* ch) {
    if (!ch) return;
    if (ch->d_st) (void)hipFree(ch->d_st);
    if (ch->d_bar) (void)hipFree(ch->d_bar);
    delete ch;
}

}  // namespace iq

// The opaque handle of include/iq.h is the library's Chain.
struct iq_chain : iq::Chain {};

extern "C" {

int iq_chain_create(const iq_stage* stages, int n, iq_chain** out) {
    iq::Chain* ch = nullptr;
    const int rc = iq::chain_create(stages, n, &ch);
    if (out) *out = static_cast<iq_chain*>(ch);
    return rc;
}

int iq_chain_run(const iq_chain* chain, void* stream) {
    if (!chain) return IQ_ENULL;
    int dev = -1;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return int(e);
    if (dev != chain->device) return IQ_EDEVICE;
    const hipError_t r = iq::chain_run(chain, static_cast<hipStream_t>(stream));
    return r == hipSuccess ? IQ_OK : int(r);
}

int iq_chain_status(const iq_chain* chain) {
    if (!chain) return IQ_ENULL;
    const hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return int(e);
    int flag = 0;
    const int rc = iq::chain_timed_out(chain, &flag);
    if (rc) return rc;
    return flag ? IQ_ETIMEOUT : IQ_OK;
}

void iq_chain_destroy(iq_chain* chain) { iq::chain_destroy(chain); }

}  // extern "C"
