// Exact parallel evaluation of the serial sum of squares s_{i+1} = RN(s_i + x_i^2) in double, i ascending
// (grad.hpp:467-473, summed per tensor by optimizer.py:66-71): the same bits as the one-lane chain, at HBM speed.
//
// Why it can be parallel. x^2 is exact in double (24 + 24 bits), so only the adds round. While s stays in one binade
// [2^e, 2^(e+1)) with ulp u = 2^(e-52), s = M u for an integer M in [2^52, 2^53), and with a = Q u + r
// (Q = floor(a / u), 0 <= r < u) the rounded sum is (M + Q + rho) u, where rho = 0 if r < u/2, 1 if r > u/2, and on a
// tie rho = 1 exactly when M + Q is odd (round half to even), valid as long as M + Q <= 2^53 - 1. So each element acts
// on (M mod 2) as a function parity -> (integer increment, new parity); these functions compose associatively, and
// a run of elements collapses to one such function. Leaving the binade, zeros at the start, non-finite values and
// any element that fails the validity bound are handled by a real double add, in order.
//
// Passes (all per fixed-size block of one tensor, blocks in index order):
//   A  block sums of x^2 (any order: an estimate only)
//   A2 per tensor, exclusive prefix of the block sums: the estimated s at each block start
//   B  per block, if the estimate puts the whole block safely inside one binade e, the block's composed function for
//      that binade (else the block is marked irregular)
//   C  per tensor, one wave walks its blocks in order with the exact s: a regular block whose binade matches the
//      exact s and whose total increment stays in the binade is applied as M += increment; anything else is walked
//      element by element with a wave-wide scan of the element functions, breaking to a real double add at the
//      first element the integer form does not cover.
// The estimate only steers speed: every application is checked against the exact state.
#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace dllm_hip {

namespace {

constexpr int kBlockElems = static_cast<int>(kSumSquaresBlock);  // 256 threads x 32 consecutive elements
constexpr int64_t kTop = (1LL << 53) - 1;

// A parity function: for incoming parity p, add d[p] to M and leave parity par[p].
struct Fn {
    long long d0, d1;
    int p0, p1;
};

__device__ __forceinline__ Fn identity_fn() { return Fn{0, 0, 0, 1}; }

// Earlier e, then later l.
__device__ __forceinline__ Fn compose(const Fn& e, const Fn& l) {
    Fn r;
    r.d0 = e.d0 + (e.p0 ? l.d1 : l.d0);
    r.p0 = e.p0 ? l.p1 : l.p0;
    r.d1 = e.d1 + (e.p1 ? l.d1 : l.d0);
    r.p1 = e.p1 ? l.p1 : l.p0;
    return r;
}

// The function of adding a (>= 0) at ulp u = 1 / inv_u; *q gets floor(a / u). Returns false when a is not finite or
// a / u >= 2^53 (the integer form does not apply).
__device__ __forceinline__ bool element_fn(double a, double inv_u, Fn* f, long long* q) {
    const double t = a * inv_u;  // exact: inv_u is a power of two and t stays a normal double
    if (!(t < 9007199254740992.0)) return false;
    const double fq = floor(t);
    const double frac = t - fq;  // exact
    const long long Q = static_cast<long long>(fq);
    const int qp = static_cast<int>(Q & 1);
    *q = Q;
    if (frac < 0.5) {
        *f = Fn{Q, Q, qp, 1 ^ qp};
    } else if (frac > 0.5) {
        *f = Fn{Q + 1, Q + 1, qp ^ 1, qp};
    } else {
        // tie: round up exactly when M + Q is odd; the result is even either way
        *f = Fn{qp ? Q + 1 : Q, qp ? Q : Q + 1, 0, 0};
    }
    return true;
}

__device__ __forceinline__ int binade(double s) {
    return static_cast<int>((static_cast<unsigned long long>(__double_as_longlong(s)) >> 52) & 0x7ff) - 1023;
}

__device__ __forceinline__ double pow2(int k) {
    return __longlong_as_double(static_cast<long long>(static_cast<unsigned long long>(k + 1023) << 52));
}

__device__ __forceinline__ Fn shfl_fn(const Fn& f, int src) {
    return Fn{__shfl(f.d0, src, 64), __shfl(f.d1, src, 64), __shfl(f.p0, src, 64), __shfl(f.p1, src, 64)};
}

__device__ __forceinline__ Fn shfl_up_fn(const Fn& f, int off) {
    return Fn{__shfl_up(f.d0, off, 64), __shfl_up(f.d1, off, 64), __shfl_up(f.p0, off, 64),
              __shfl_up(f.p1, off, 64)};
}

__device__ __forceinline__ Fn shfl_down_fn(const Fn& f, int off) {
    return Fn{__shfl_down(f.d0, off, 64), __shfl_down(f.d1, off, 64), __shfl_down(f.p0, off, 64),
              __shfl_down(f.p1, off, 64)};
}

__device__ __forceinline__ long long readlane64(long long v, int k) {
    const int lo = __builtin_amdgcn_readlane(static_cast<int>(v & 0xffffffffLL), k);
    const int hi = __builtin_amdgcn_readlane(static_cast<int>(v >> 32), k);
    return (static_cast<long long>(hi) << 32) | static_cast<unsigned int>(lo);
}

__device__ __forceinline__ double sq(float x) { return static_cast<double>(x) * static_cast<double>(x); }

__device__ __forceinline__ double infinity() { return __longlong_as_double(0x7ff0000000000000LL); }

// The function of elements x[i0, i0 + n) (n <= 32) in order at ulp 1 / inv_u; false if one of them is outside the
// integer form.
__device__ __forceinline__ bool run_fn(const float* __restrict__ x, int64_t i0, int n, double inv_u, Fn* f) {
    Fn r = identity_fn();
    bool ok = true;
    if (n == 32 && reinterpret_cast<uintptr_t>(x + i0) % 16 == 0) {
        float v[32];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float4 q4 = reinterpret_cast<const float4*>(x + i0)[k];
            v[4 * k] = q4.x;
            v[4 * k + 1] = q4.y;
            v[4 * k + 2] = q4.z;
            v[4 * k + 3] = q4.w;
        }
#pragma unroll
        for (int k = 0; k < 32; ++k) {
            Fn g;
            long long q;
            ok = ok && element_fn(sq(v[k]), inv_u, &g, &q);
            r = compose(r, g);
        }
    } else {
        for (int k = 0; k < n; ++k) {
            Fn g;
            long long q;
            ok = ok && element_fn(sq(x[i0 + k]), inv_u, &g, &q);
            r = compose(r, g);
        }
    }
    *f = r;
    return ok;
}

// The exact serial chain over x[begin, end) from state s, with the 64 lanes of one wave (all lanes call it with the
// same arguments; all return the same s).
//
// Coarse steps first: 2048 elements at once, 32 consecutive per lane composed in order, then scanned in lane order.
// The state only grows, so a lane's run is covered when the state after it is at most 2^53 - 1 (each M_j + Q_j is
// at most the next M). The lanes before the first uncovered run are applied at once; that run goes to the fine steps
// below (64 elements at a time, up to the element that needs a real add), then the coarse steps resume.
__device__ double walk(const float* __restrict__ x, int64_t begin, int64_t end, double s) {
    const int lane = static_cast<int>(threadIdx.x) & 63;
    int64_t i = begin;
    int64_t fine_until = begin;  // the fine steps take [i, fine_until): a coarse run failed there
    while (i < end) {
        if (i >= fine_until && end - i >= 2048 && s == s && s > 0.0 && s < infinity()) {
            const int e = binade(s);
            const double inv_u = pow2(52 - e);
            const long long M = static_cast<long long>(s * inv_u);
            const int p = static_cast<int>(M & 1);
            Fn f;
            const bool ok = run_fn(x, i + 32 * lane, 32, inv_u, &f);
            // inclusive scan in lane order: lane k's state after its run
            Fn inc = f;
            for (int off = 1; off < 64; off <<= 1) {
                const Fn g = shfl_up_fn(inc, off);
                if (lane >= off) inc = compose(g, inc);
            }
            const long long after = M + (p ? inc.d1 : inc.d0);
            // the first lane whose run is not covered (a value outside the integer form, or the state past the
            // binade); the lanes before it are applied at once
            const unsigned long long bad = __ballot(!ok || after > kTop);
            if (bad == 0) {
                s = static_cast<double>(readlane64(after, 63)) * pow2(e - 52);
                i += 2048;
                continue;
            }
            const int k = __ffsll(static_cast<long long>(bad)) - 1;
            if (k > 0) {
                s = static_cast<double>(readlane64(after, k - 1)) * pow2(e - 52);
                i += 32 * k;
            }
            fine_until = i + 32;  // the fine steps take the run that is not covered
        }
        const int64_t idx = i + lane;
        const double a = idx < end ? sq(x[idx]) : 0.0;
        if (s != s) return s;  // NaN absorbs everything
        if (s == infinity()) {
            // inf + finite = inf; inf + NaN = NaN
            const unsigned long long nan_lanes = __ballot(a != a);
            if (nan_lanes) return __shfl(a, __ffsll(static_cast<long long>(nan_lanes)) - 1, 64);
            i += 64;
            continue;
        }
        if (s == 0.0) {
            // leading zeros keep s = +0; the first non-zero element becomes s exactly. Runs of 2048 zeros at a time
            // first (a square is zero only for +-0: the smallest float squared is a normal double)
            if (end - i >= 2048 + 64) {
                bool zero = true;
                const float* r = x + i + 64 + 32 * lane;
                for (int k = 0; k < 32; ++k) zero = zero && r[k] == 0.0f;
                if (__ballot(!zero) == 0 && __ballot(a != 0.0) == 0) {
                    i += 2048 + 64;
                    continue;
                }
            }
            const unsigned long long nz = __ballot(a != 0.0);
            if (nz == 0) {
                i += 64;
                continue;
            }
            const int k = __ffsll(static_cast<long long>(nz)) - 1;
            s = s + __shfl(a, k, 64);
            i += k + 1;
            continue;
        }
        const int e = binade(s);
        const double inv_u = pow2(52 - e);
        const double u = pow2(e - 52);
        const long long M = static_cast<long long>(s * inv_u);
        const int p = static_cast<int>(M & 1);
        Fn f = identity_fn();
        long long q = 0;
        bool ok = element_fn(a, inv_u, &f, &q);
        // inclusive scan in lane order
        Fn inc = f;
        for (int off = 1; off < 64; off <<= 1) {
            const Fn g = shfl_up_fn(inc, off);
            if (lane >= off) inc = compose(g, inc);
        }
        Fn ex = shfl_up_fn(inc, 1);
        if (lane == 0) ex = identity_fn();
        const long long Mj = M + (p ? ex.d1 : ex.d0);
        const bool bad = idx < end && (!ok || Mj + q > kTop);
        const unsigned long long bad_lanes = __ballot(bad);
        if (bad_lanes == 0) {
            const Fn all = shfl_fn(inc, 63);
            s = static_cast<double>(M + (p ? all.d1 : all.d0)) * u;
            i += 64;
            continue;
        }
        const int k = __ffsll(static_cast<long long>(bad_lanes)) - 1;
        const Fn before = shfl_fn(ex, k);
        s = static_cast<double>(M + (p ? before.d1 : before.d0)) * u;
        s = s + __shfl(a, k, 64);  // the reference's own add for the element the integer form does not cover
        i += k + 1;
        fine_until = i;  // past the element that needed a real add: coarse steps again
    }
    return s;
}

struct BlockRec {
    long long d0, d1;
    int p0, p1;
    int e;
    int regular;
};

// Pass A: the sum of a block's squares, in any order (an estimate).
__global__ __launch_bounds__(256) void block_sums_kernel(const float* __restrict__ arena,
                                                         const int64_t* __restrict__ bstart,
                                                         const int64_t* __restrict__ bcount,
                                                         double* __restrict__ bsum) {
    __shared__ double part[256];
    const int64_t b = blockIdx.x;
    const float* x = arena + bstart[b];
    const int64_t n = bcount[b];
    double acc = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += 256) acc += sq(x[i]);
    part[threadIdx.x] = acc;
    __syncthreads();
    for (int w = 128; w >= 1; w >>= 1) {
        if (static_cast<int>(threadIdx.x) < w) part[threadIdx.x] += part[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) bsum[b] = part[0];
}

// Pass A2: per tensor (one wave), exclusive prefix of its block sums.
__global__ __launch_bounds__(64) void block_prefix_kernel(const int64_t* __restrict__ tfirst,
                                                          const int64_t* __restrict__ tblocks,
                                                          const double* __restrict__ bsum, double* __restrict__ est) {
    const int64_t t = blockIdx.x;
    const int lane = threadIdx.x;
    const int64_t b0 = tfirst[t], nb = tblocks[t];
    double carry = 0.0;
    for (int64_t c = 0; c < nb; c += 64) {
        const double v = c + lane < nb ? bsum[b0 + c + lane] : 0.0;
        double inc = v;
        for (int off = 1; off < 64; off <<= 1) {
            const double g = __shfl_up(inc, off, 64);
            if (lane >= off) inc += g;
        }
        if (c + lane < nb) est[b0 + c + lane] = carry + (inc - v);
        carry += __shfl(inc, 63, 64);
    }
}

// Pass B: the composed function of a block for the binade its estimated start and end share, if they safely do.
__global__ __launch_bounds__(256) void block_fn_kernel(const float* __restrict__ arena,
                                                       const int64_t* __restrict__ bstart,
                                                       const int64_t* __restrict__ bcount,
                                                       const double* __restrict__ bsum,
                                                       const double* __restrict__ est, BlockRec* __restrict__ rec) {
    __shared__ Fn wave_fn[4];
    __shared__ int wave_ok[4];
    const int64_t b = blockIdx.x;
    const double lo = est[b] * (1.0 - 1e-5), hi = (est[b] + bsum[b]) * (1.0 + 1e-5);
    const bool plausible = lo > 2.2250738585072014e-308 && hi < 1e300 && binade(lo) == binade(hi);
    if (!plausible) {
        if (threadIdx.x == 0) rec[b] = BlockRec{0, 0, 0, 1, 0, 0};
        return;  // block-uniform
    }
    const int e = binade(lo);
    const double inv_u = pow2(52 - e);
    const float* x = arena + bstart[b];
    const int64_t n = bcount[b];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // each thread composes its 32 consecutive elements in order
    Fn f = identity_fn();
    bool ok = true;
    const int64_t i0 = static_cast<int64_t>(tid) * 32;
    if (i0 + 32 <= n && reinterpret_cast<uintptr_t>(x + i0) % 16 == 0) {
        // a whole run: 8 vector loads, then the 32 elements in order
        float v[32];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float4 q4 = reinterpret_cast<const float4*>(x + i0)[k];
            v[4 * k] = q4.x;
            v[4 * k + 1] = q4.y;
            v[4 * k + 2] = q4.z;
            v[4 * k + 3] = q4.w;
        }
        for (int k = 0; k < 32; ++k) {
            Fn g;
            long long q;
            ok = ok && element_fn(sq(v[k]), inv_u, &g, &q);
            f = compose(f, g);
        }
    } else {
        for (int k = 0; k < 32; ++k) {
            const int64_t i = i0 + k;
            if (i >= n) break;
            Fn g;
            long long q;
            ok = ok && element_fn(sq(x[i]), inv_u, &g, &q);
            f = compose(f, g);
        }
    }
    // ordered reduction over the wave's lanes
    for (int off = 1; off < 64; off <<= 1) {
        const Fn g = shfl_down_fn(f, off);
        if ((lane & (2 * off - 1)) == 0) f = compose(f, g);
    }
    const bool wave_all_ok = __ballot(!ok) == 0;
    if (lane == 0) {
        wave_fn[wave] = f;
        wave_ok[wave] = wave_all_ok;
    }
    __syncthreads();
    if (tid == 0) {
        Fn total = wave_fn[0];
        int good = wave_ok[0];
        for (int w = 1; w < 4; ++w) {
            total = compose(total, wave_fn[w]);
            good &= wave_ok[w];
        }
        rec[b] = BlockRec{total.d0, total.d1, total.p0, total.p1, e, good};
    }
}

// Pass C: per tensor, the exact walk over its blocks. The lanes load the records of 64 blocks at a time and the walk
// takes block k's fields from lane k. While consecutive regular blocks share a binade e the state stays the integer
// M (s = M 2^(e-52), M in [2^52, 2^53)): after an application M + tot <= 2^53 - 1 and tot >= 0, so s stays in
// binade e and the next block's M = s 2^(52-e) is that same integer. s is formed only when the walk leaves that path.

__global__ __launch_bounds__(64) void tensor_walk_kernel(const float* __restrict__ arena,
                                                         const int64_t* __restrict__ tfirst,
                                                         const int64_t* __restrict__ tblocks,
                                                         const int64_t* __restrict__ bstart,
                                                         const int64_t* __restrict__ bcount,
                                                         const BlockRec* __restrict__ rec,
                                                         const double* __restrict__ bsum,
                                                         double* __restrict__ per_tensor) {
    const int64_t t = blockIdx.x;
    const int lane = static_cast<int>(threadIdx.x);
    const int64_t b0 = tfirst[t], nb = tblocks[t];
    double s = 0.0;
    bool have = false;  // s == M 2^(e - 52)
    long long M = 0;
    int e = 0;
    for (int64_t bc = b0; bc < b0 + nb; bc += 64) {
        const BlockRec mine = bc + lane < b0 + nb ? rec[bc + lane] : BlockRec{0, 0, 0, 1, 0, 0};
        const int cnt = static_cast<int>(b0 + nb - bc < 64 ? b0 + nb - bc : 64);
        // the 64 blocks at once when all are regular in the current binade: their functions compose in order, and
        // since increments are non-negative, the whole run's bound covers every block's
        if (have && __ballot(lane < cnt && !(mine.regular && mine.e == e)) == 0) {
            Fn f = lane < cnt ? Fn{mine.d0, mine.d1, mine.p0, mine.p1} : identity_fn();
            for (int off = 1; off < 64; off <<= 1) {
                const Fn g = shfl_down_fn(f, off);
                if ((lane & (2 * off - 1)) == 0) f = compose(f, g);
            }
            const long long tot = (M & 1) ? readlane64(f.d1, 0) : readlane64(f.d0, 0);
            if (M + tot <= kTop) {
                M += tot;
                continue;
            }
        }
        for (int k = 0; k < cnt; ++k) {
            const int regular = __builtin_amdgcn_readlane(mine.regular, k);
            const int re = __builtin_amdgcn_readlane(mine.e, k);
            const long long d0 = readlane64(mine.d0, k), d1 = readlane64(mine.d1, k);
            if (have && regular && re == e) {
                const long long tot = (M & 1) ? d1 : d0;
                if (M + tot <= kTop) {
                    M += tot;
                    continue;
                }
            }
            if (have) {
                s = static_cast<double>(M) * pow2(e - 52);
                have = false;
            }
            if (regular && s > 0.0 && s < infinity() && binade(s) == re) {
                const long long M0 = static_cast<long long>(s * pow2(52 - re));
                const long long tot = (M0 & 1) ? d1 : d0;
                if (M0 + tot <= kTop) {
                    M = M0 + tot;
                    e = re;
                    have = true;
                    continue;
                }
            }
            const int64_t b = bc + k;
            if (s == 0.0 && bsum[b] == 0.0) continue;  // a block of zeros keeps s = +0 (its squares are exact)
            s = walk(arena, bstart[b], bstart[b] + bcount[b], s);
        }
    }
    if (have) s = static_cast<double>(M) * pow2(e - 52);
    if (threadIdx.x == 0) per_tensor[t] = s;
}

}  // namespace

size_t exact_sum_squares_blocks(const int64_t* counts, int64_t tensors) {
    size_t blocks = 0;
    for (int64_t t = 0; t < tensors; ++t) blocks += ceil_div(static_cast<size_t>(counts[t] > 0 ? counts[t] : 1), kBlockElems);
    return blocks;
}

void exact_sum_squares_plan(const int64_t* offsets, const int64_t* counts, int64_t tensors, int64_t* tfirst,
                            int64_t* tblocks, int64_t* bstart, int64_t* bcount) {
    int64_t b = 0;
    for (int64_t t = 0; t < tensors; ++t) {
        tfirst[t] = b;
        const int64_t n = counts[t];
        const int64_t nb = n > 0 ? (n + kBlockElems - 1) / kBlockElems : 1;
        tblocks[t] = nb;
        for (int64_t k = 0; k < nb; ++k) {
            bstart[b] = offsets[t] + k * kBlockElems;
            bcount[b] = n > 0 ? std::min<int64_t>(kBlockElems, n - k * kBlockElems) : 0;
            ++b;
        }
    }
}

size_t exact_sum_squares_workspace(size_t blocks) {
    return blocks * (2 * sizeof(double) + sizeof(BlockRec)) + 256;
}

int launch_exact_sum_squares(const float* arena, const ExactSumPlan& plan, void* workspace, double* per_tensor,
                             hipStream_t stream) {
    if (plan.tensors == 0) return kOk;
    double* bsum = static_cast<double*>(workspace);
    double* est = bsum + plan.blocks;
    BlockRec* rec = reinterpret_cast<BlockRec*>(est + plan.blocks);
    const unsigned nb = static_cast<unsigned>(plan.blocks);
    const unsigned nt = static_cast<unsigned>(plan.tensors);
    hipLaunchKernelGGL(block_sums_kernel, dim3(nb), dim3(256), 0, stream, arena, plan.bstart, plan.bcount, bsum);
    DLLM_TRY(check_launch("sum_squares pass A"));
    hipLaunchKernelGGL(block_prefix_kernel, dim3(nt), dim3(64), 0, stream, plan.tfirst, plan.tblocks, bsum, est);
    DLLM_TRY(check_launch("sum_squares pass A2"));
    hipLaunchKernelGGL(block_fn_kernel, dim3(nb), dim3(256), 0, stream, arena, plan.bstart, plan.bcount, bsum, est,
                       rec);
    DLLM_TRY(check_launch("sum_squares pass B"));
    hipLaunchKernelGGL(tensor_walk_kernel, dim3(nt), dim3(64), 0, stream, arena, plan.tfirst, plan.tblocks,
                       plan.bstart, plan.bcount, rec, bsum, per_tensor);
    return check_launch("sum_squares pass C");
}

}  // namespace dllm_hip
