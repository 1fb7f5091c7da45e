// wkv7_oracle.cpp -- CPU restatement of the RWKV-7 WKV recurrence.
//
// TEST INFRASTRUCTURE ONLY.  Nothing in the product path links, loads or calls this file: only tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the checker or as the timed CPU baseline.
// The HIP library fails loudly when its own build is missing; it never falls back to this code.
//
// Semantics restated from the reference (OpenMOSE/RWKV-Infer-Next):
//   rwkv_next/kernels/wkv7.py:4-7    S_t = diag(d_t) S_{t-1} + b_t (a_t^T S_{t-1}) + k_t v_t^T,  o_t = S_t^T r_t
//   rwkv_next/kernels/wkv7.py:46-52  varlen: bos = cu[n], L = cu[n+1]-cu[n]; dense: bos = n*T, L = T
//   rwkv_next/kernels/wkv7.py:53-54  L = min(L, n_keep[n])
//   rwkv_next/kernels/wkv7.py:62-64  S = h0[n] (fp32) or zeros
//   rwkv_next/kernels/wkv7.py:65-77  per step: d = exp(-exp(w)) from the RAW w; the a^T S term and the decay
//                                    both use the OLD state; o_t is taken from the UPDATED state
//   rwkv_next/kernels/wkv7.py:78-79  ht[n] = S
//   tools/test_wkv7.py:13-23         fp64 loop, sums over the k axis
//
// Layouts are the reference's: operands r, w, k, v, a, b are [tokens][H][K] (token stride H*K), passed here as
// float32 holding the bf16-rounded values; states are [seq][H][K][V] with V contiguous (K == V <= 256: the reference
// takes any head size, padding it to a power of two with masks, wkv7.py:55-59, 96).
//
// Two precisions: wkv7_oracle_f64 (the parity reference) and wkv7_oracle_f32 (the timed CPU baseline and the
// fp32-vs-fp64 calibration of the tolerances).  Both parallelise over (sequence, head) pairs with OpenMP; the
// arithmetic order inside a pair is fixed and does not depend on the thread count.
//
// Parity pins (tests/test_oracle.py): closed forms -- pure accumulation (cumulative sum of outer products),
// decayed linear attention (masked matmul), pure decay, the I - kappa kappa^T projector, an asymmetric
// elementary row operation for the b (a^T S) orientation, and explicit transition-matrix products; invariants --
// varlen == per-sequence, chunk associativity, n_keep == prefix run, snapshots == prefix states.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>
#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

constexpr int KMAX = 256;

// Sequence extents, rwkv_next/kernels/wkv7.py:46-54.
inline void seq_extent(int n, int T, const int32_t* cu, const int64_t* nkeep, int64_t* bos, int64_t* len) {
    if (cu) {
        *bos = cu[n];
        *len = (int64_t)cu[n + 1] - cu[n];
    } else {
        *bos = (int64_t)n * T;
        *len = T;
    }
    if (nkeep && nkeep[n] < *len) *len = nkeep[n];
    if (*len < 0) *len = 0;
}

inline double exp_of(double x) { return std::exp(x); }
inline float exp_of(float x) { return std::exp(x); }

template <typename Real>
int run(const float* r, const float* w, const float* k, const float* v, const float* a, const float* b, Real* o,
        const float* h0, const int64_t* state_idx, Real* ht, const int32_t* cu, const int64_t* nkeep, Real* snap,
        int num_seqs, int T, int H, int K, int nthreads) {
    if (num_seqs < 0 || T < 0 || H <= 0 || K <= 0 || K > KMAX) return -1;
    const int64_t ts = (int64_t)H * K;  // token stride
    const int64_t KK = (int64_t)K * K;
    const int npairs = num_seqs * H;
    const int nt = nthreads > 0 ? nthreads : 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
    for (int p = 0; p < npairs; ++p) {
        const int n = p / H, h = p % H;
        int64_t bos, L;
        seq_extent(n, T, cu, nkeep, &bos, &L);
        const int64_t slot = state_idx ? state_idx[n] : n;
        std::vector<Real> Sv(KK), sav(K), ddv(K);  // per pair on the heap (K up to 256)
        Real *S = Sv.data(), *sa = sav.data(), *dd = ddv.data();
        if (h0) {
            const float* s0 = h0 + (slot * H + h) * KK;
            for (int64_t i = 0; i < KK; ++i) S[i] = (Real)s0[i];
        } else {
            for (int64_t i = 0; i < KK; ++i) S[i] = 0;
        }
        for (int64_t t = 0; t < L; ++t) {
            const int64_t off = (bos + t) * ts + (int64_t)h * K;
            const float *rr = r + off, *ww = w + off, *kk = k + off, *vv = v + off, *aa = a + off, *bb = b + off;
            // sa[j] = sum_i a_i S[i][j] over the OLD state (wkv7.py:75, tl.sum over axis 0)
            for (int j = 0; j < K; ++j) sa[j] = 0;
            for (int i = 0; i < K; ++i) {
                const Real ai = (Real)aa[i];
                for (int j = 0; j < K; ++j) sa[j] += ai * S[i * K + j];
            }
            // d = exp(-exp(w)) from the raw w (wkv7.py:74)
            for (int i = 0; i < K; ++i) dd[i] = exp_of(-exp_of((Real)ww[i]));
            // S[i][j] = d_i S[i][j] + b_i sa[j] + k_i v_j (wkv7.py:75)
            for (int i = 0; i < K; ++i) {
                const Real di = dd[i], bi = (Real)bb[i], ki = (Real)kk[i];
                for (int j = 0; j < K; ++j) S[i * K + j] = di * S[i * K + j] + bi * sa[j] + ki * (Real)vv[j];
            }
            // o_t[j] = sum_i S[i][j] r_i from the UPDATED state (wkv7.py:76-77)
            if (o) {
                Real* out = o + off;
                for (int j = 0; j < K; ++j) {
                    Real acc = 0;
                    for (int i = 0; i < K; ++i) acc += S[i * K + j] * (Real)rr[i];
                    out[j] = acc;
                }
            }
            if (snap) {
                Real* sp = snap + (((int64_t)n * T + t) * H + h) * KK;
                std::memcpy(sp, S, sizeof(Real) * KK);
            }
        }
        if (ht) std::memcpy(ht + (slot * H + h) * KK, S, sizeof(Real) * KK);
    }
    return 0;
}

}  // namespace

extern "C" {

// All pointers are host pointers.  o, ht, snap are nullable outputs; h0 is a nullable fp32 initial-state array
// indexed by state_idx[n] (a pool slot) when state_idx is given, else by n; ht is indexed the same way.
// snap is [num_seqs][T][H][K][K]: the state after each token (rows past a sequence's length are not written).
// Returns 0, or -1 for invalid sizes (K > 256).
int wkv7_oracle_f64(const float* r, const float* w, const float* k, const float* v, const float* a, const float* b,
                    double* o, const float* h0, const int64_t* state_idx, double* ht, const int32_t* cu,
                    const int64_t* nkeep, double* snap, int num_seqs, int T, int H, int K, int nthreads) {
    return run<double>(r, w, k, v, a, b, o, h0, state_idx, ht, cu, nkeep, snap, num_seqs, T, H, K, nthreads);
}

int wkv7_oracle_f32(const float* r, const float* w, const float* k, const float* v, const float* a, const float* b,
                    float* o, const float* h0, const int64_t* state_idx, float* ht, const int32_t* cu,
                    const int64_t* nkeep, float* snap, int num_seqs, int T, int H, int K, int nthreads) {
    return run<float>(r, w, k, v, a, b, o, h0, state_idx, ht, cu, nkeep, snap, num_seqs, T, H, K, nthreads);
}

int wkv7_oracle_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

}  // extern "C"
