// k_fold.hip -- the decode step's Wdown of layer l and Wqkv of layer l+1 in
// one launch (model.c:728-736, then 338-345 and 711-722 of the next layer).
//
// Every wave issues its Wdown row group's weights and right behind them its
// Wqkv row group's, computes the Wdown rows as k_gemv does for one token with
// the fp32 h quantized to q8_0 in the workgroup (the same lanes, units and
// reduction, so each row keeps the bits of that launch), stores them and
// publishes them as tagged words.  Every workgroup then polls all Wdown rows,
// applies the residual update and RMSNorm of the persistent family's PRO_NORM
// prologue (run by the first 512 threads with that family's slots, so its
// sums and bits are those of the separate launch), quantizes to q8_0 in LDS
// and finishes its Wqkv rows with k_gemv_p's lanes, units and reduction.  One
// launch instead of two, every output bit-identical to the separate kernels;
// measured slower than the two launches (the gather of the rows waits for
// round trips behind the other CUs' streams), so the decode step runs it only
// on request (G4H_DECODE_FUSE bit 64).
//
// The grid is sized so that every workgroup is resident at once (it polls the
// others' rows); a poll gives up after a bounded number of retries, writes
// NaN into its Wqkv rows and sets the error word, so the launch always ends.
#include "formats.h"
#include "gemv_p.h"
#include "handoff.h"
#include "kernels.h"

#include <map>
#include <mutex>

namespace g4 {

struct DqArgs {
    g4h_tensor Wd, Wq;
    const float *h;          // [Wd.ncols] fp32 input of Wdown
    float *yd;               // [Wd.nrows] Wdown rows (the branch output delta)
    uint64_t *words;         // the same rows as tagged words, wstride per workgroup
    GemvPro pro;             // Wqkv's PRO_NORM prologue (delta taken from the words)
    float *yq;               // [Wq.nrows]
    const unsigned *epoch;   // this launch's tag is *epoch * tag_mul + tag_add + 1
    unsigned tag_mul, tag_add;
    unsigned *err;           // set when a poll gives up
    unsigned spin;
    uint32_t poll_xor;       // test hook: polls wait for a tag no store carries
    int units_d, units_q;
    int wstride;             // words per workgroup: its rows in lines of their own
    uint32_t lds_q, lds_x;   // byte offsets of Wqkv's activation and the gathered rows
};

template <class FD, int LPRD, int UPLD, class FQ, int LPRQ, int UPLQ, int S>
__global__ __launch_bounds__(1024) void k_down_qkv(DqArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int bad;
    uint8_t *lds_d = lds, *lds_q = lds + a.lds_q;
    float *dl = (float *)(lds + a.lds_x);
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, nwv = (int)(blockDim.x >> 6);
    const uint32_t tag = *a.epoch * a.tag_mul + a.tag_add + 1u;
    if (t == 0) bad = 0;
    constexpr int PBD = 64 * GP_WAVES;                               // the persistent family's prologue threads

    // Wqkv's prologue inputs first (small loads ahead of the streams)
    ProLoads pr;
    pro_issue<PRO_NORM, S>(pr, a.pro, PBD, false);
    // Wdown as k_gemv with the fp32 input quantized in the workgroup (four
    // groups of 4 per thread)
    constexpr int RPWD = 64 / LPRD;
    const int gd = lane % LPRD, rgd = lane / LPRD;
    const int64_t rowd0 = ((int64_t)blockIdx.x * nwv + wave) * RPWD + rgd;
    const bool rowd_ok = rowd0 < a.Wd.nrows;
    const int64_t rowd = rowd_ok ? rowd0 : a.Wd.nrows - 1;
    const int gpt = (int)(a.Wd.ncols >> 2);
    float xv[4][4];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int gi = min((int)(t + s * blockDim.x), gpt - 1);
        const float4 v = *(const float4 *)(a.h + 4 * (size_t)gi);
        xv[s][0] = v.x; xv[s][1] = v.y; xv[s][2] = v.z; xv[s][3] = v.w;
    }
    issue_barrier();
    typename FD::Frag fd[UPLD];
#pragma unroll
    for (int k = 0; k < UPLD; k++) FD::load(fd[k], a.Wd, rowd, min(gd + k * LPRD, a.units_d - 1));
    // Wqkv: this wave's row group streams right behind Wdown's
    constexpr int RPWQ = 64 / LPRQ;
    const int gq = lane % LPRQ, rgq = lane / LPRQ;
    const int64_t grq = (int64_t)blockIdx.x * nwv + wave;
    const int64_t rowq0 = grq * RPWQ + rgq;
    const int64_t rowq = min(rowq0, a.Wq.nrows - 1);
    typename FQ::Frag fq[UPLQ];
#pragma unroll
    for (int k = 0; k < UPLQ; k++) FQ::load(fq[k], a.Wq, rowq, min(gq + k * LPRQ, a.units_q - 1));
    issue_order();
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int gi = t + s * blockDim.x;
        q8_lds4(xv[s], gi, gi < gpt, lds_d, (int)a.Wd.nb, 0);
    }
    lds_barrier();
    float acc = 0.0f;
    {
        const ActQ8_0 A(lds_d, (int)a.Wd.nb, 0);
#pragma unroll
        for (int k = 0; k < UPLD; k++) {
            const int u = gd + k * LPRD;
            if (u < a.units_d) acc = FD::accum(fd[k], A, u, acc);
        }
    }
    acc = group_sum<LPRD>(acc);

    // publish this wave's Wdown rows (a workgroup's rows share lines written
    // by that workgroup alone: lines shared by writers on other CUs were seen
    // to carry their last store late), then gather all of them
    const int rpwg = nwv * RPWD;                                     // rows per workgroup
    if (gd == 0 && rowd_ok) {
        a.yd[rowd0] = acc;
        st_tag(a.words + (size_t)blockIdx.x * a.wstride + (rowd0 - (int64_t)blockIdx.x * rpwg), __float_as_uint(acc), tag);
    }
    const int nd = (int)a.Wd.nrows;
    for (int i0 = 0; i0 < nd; i0 += 4 * (int)blockDim.x) {           // uniform
        const uint64_t *src[4];
        bool need[4];
        uint32_t bits[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int i = i0 + q * (int)blockDim.x + t, ic = min(i, nd - 1);
            src[q] = a.words + (size_t)(ic / rpwg) * a.wstride + ic % rpwg;
            need[q] = i < nd;
        }
        if (!poll_words<4>(src, need, tag ^ a.poll_xor, bits, a.spin)) bad = 1;
#pragma unroll
        for (int q = 0; q < 4; q++)
            if (need[q]) dl[i0 + q * (int)blockDim.x + t] = __uint_as_float(bits[q]);
    }
    lds_barrier();
    // the prologue's delta from the gathered rows, then the norm and q8_0
    {
        const int ng = a.pro.n >> 2;
#pragma unroll
        for (int s = 0; s < S; s++) {
            const int gi = t + s * PBD;
            if (t < PBD && gi < ng) {
#pragma unroll
                for (int k = 0; k < 4; k++) pr.d[s][k] = dl[4 * gi + k];
            }
        }
    }
    pro_finish<PRO_NORM, S>(pr, a.pro, lds_q, (int)a.Wq.nb, blockIdx.x == 0, PBD);
    lds_barrier();
    float accq = 0.0f;
    {
        const ActQ8_0 A(lds_q, (int)a.Wq.nb, 0);
#pragma unroll
        for (int k = 0; k < UPLQ; k++) {
            const int u = gq + k * LPRQ;
            if (u < a.units_q) accq = FQ::accum(fq[k], A, u, accq);
        }
    }
    accq = group_sum<LPRQ>(accq);
    const int64_t ngq = (a.Wq.nrows + RPWQ - 1) / RPWQ;
    if (grq < ngq && gq == 0 && rowq0 < a.Wq.nrows) a.yq[rowq0] = bad ? __builtin_nanf("") : accq;
    lds_barrier();
    if (t == 0 && bad) st_ag(a.err, 1u);
}

namespace {

// the launch shape: the LPR / UPL of each matrix as its separate launch takes
// them, the prologue slots, waves per workgroup and the grid
struct DqShape {
    int lprd, upld, lprq, uplq, s, nwv, wstride;
    int64_t grid;
    size_t words, lds, lds_q, lds_x;
};

bool dq_shape(const g4h_tensor &Wd, const g4h_tensor &Wq, DqShape *sh) {
    if (Wd.type != Wq.type || (Wd.type != Q4_0 && Wd.type != Q8_0)) return false;
    if (Wd.ncols % 16 || Wq.ncols % 4 || Wq.ncols != Wd.nrows) return false;
    int l, u;
    gemv_shape(Wd.type, Wd.nb, &l, &u);
    sh->lprd = l;
    sh->upld = gemv_upl_final(Wd.type, Wd.nb, 1, l, u);
    gemv_shape(Wq.type, Wq.nb, &l, &u);
    sh->lprq = l;
    sh->uplq = gemv_upl_final(Wq.type, Wq.nb, 1, l, u);
    if ((int64_t)sh->lprd * sh->upld < Wd.nb || (int64_t)sh->lprq * sh->uplq < Wq.nb) return false;   // one pass per row
    const int slots = (int)((Wq.ncols / 4 + 64 * GP_WAVES - 1) / (64 * GP_WAVES));
    if (slots > 2) return false;                                     // the instantiated prologue: S = 2
    sh->s = 2;
    const int64_t gpt = Wd.ncols / 4;
    int nwv = (int)((gpt + 4 * 64 - 1) / (4 * 64));                   // four groups of 4 per thread
    if (nwv < GP_WAVES) nwv = GP_WAVES;                              // the prologue's 512 threads
    if (nwv > 16) return false;
    sh->nwv = nwv;
    const int64_t waves_d = (Wd.nrows + 64 / sh->lprd - 1) / (64 / sh->lprd);
    const int64_t groups_q = (Wq.nrows + 64 / sh->lprq - 1) / (64 / sh->lprq);
    sh->grid = (std::max(waves_d, groups_q) + nwv - 1) / nwv;
    const int rpwg = nwv * (64 / sh->lprd);
    sh->wstride = (rpwg + 15) & ~15;                                  // whole 128-byte lines per workgroup
    sh->words = (size_t)sh->grid * sh->wstride;
    const size_t ad = (ActQ8_0::bytes_per_token((int)Wd.nb) + 15) & ~(size_t)15;
    const size_t aq = (ActQ8_0::bytes_per_token((int)Wq.nb) + 15) & ~(size_t)15;
    sh->lds_q = ad;
    sh->lds_x = ad + aq;
    sh->lds = ad + aq + (size_t)Wd.nrows * 4;
    return sh->lds <= 64 * 1024;
}

template <class F, int LD, int UD, int LQ, int UQ>
const void *dq_kernel() {
    return reinterpret_cast<const void *>(k_down_qkv<F, LD, UD, F, LQ, UQ, 2>);
}

// the instantiated shapes: the BASELINE model's q4_0 / q8_0 FFN and
// projection widths (Wdown 64 x 5, Wqkv 32 x 3 or 64 x 2) and small test
// models (16 x 1 .. 16 x 2)
const void *dq_pick(const g4h_tensor &Wd, const DqShape &sh) {
#define G4_DQ(F, LD, UD, LQ, UQ) \
    if (sh.lprd == LD && sh.upld == UD && sh.lprq == LQ && sh.uplq == UQ) return dq_kernel<F, LD, UD, LQ, UQ>()
    if (Wd.type == Q4_0) {
        G4_DQ(FQ4_0, 64, 5, 32, 3); G4_DQ(FQ4_0, 64, 5, 64, 2); G4_DQ(FQ4_0, 16, 1, 16, 1); G4_DQ(FQ4_0, 16, 2, 16, 1);
        G4_DQ(FQ4_0, 16, 1, 16, 2); G4_DQ(FQ4_0, 16, 2, 16, 2);
    } else {
        G4_DQ(FQ8_0, 64, 5, 32, 3); G4_DQ(FQ8_0, 64, 5, 64, 2); G4_DQ(FQ8_0, 16, 1, 16, 1); G4_DQ(FQ8_0, 16, 2, 16, 1);
        G4_DQ(FQ8_0, 16, 1, 16, 2); G4_DQ(FQ8_0, 16, 2, 16, 2);
    }
#undef G4_DQ
    return nullptr;
}

// workgroups of this kernel and shape the device holds resident at once
int dq_capacity(const void *kernel, int threads, size_t lds) {
    static std::mutex mu;
    static std::map<std::pair<const void *, std::pair<int, size_t>>, int> cache;
    std::lock_guard<std::mutex> lk(mu);
    const auto key = std::make_pair(kernel, std::make_pair(threads, lds));
    const auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int dev = 0, cus = 0, occ = 0, cap = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, threads, lds) == hipSuccess)
        cap = cus * occ;
    cache[key] = cap;
    return cap;
}

}  // namespace

bool down_qkv_fits(const g4h_tensor &Wd, const g4h_tensor &Wq, const GemvPro &pro, size_t words) {
    DqShape sh;
    if (pro.kind != PRO_NORM || pro.n != Wq.ncols || !dq_shape(Wd, Wq, &sh) || sh.words > words) return false;
    const void *k = dq_pick(Wd, sh);
    return k && sh.grid <= dq_capacity(k, 64 * sh.nwv, sh.lds);
}

hipError_t launch_down_qkv(const g4h_tensor &Wd, const float *h, float *yd, uint64_t *words, size_t nwords, const g4h_tensor &Wq,
                           const GemvPro &pro, float *yq, const AttnTag &tag, unsigned *err, hipStream_t s) {
    if (!down_qkv_fits(Wd, Wq, pro, nwords) || !h || !yd || !words || !yq || !err || !tag.epoch || (uintptr_t)h % 16)
        return hipErrorInvalidValue;
    DqShape sh;
    dq_shape(Wd, Wq, &sh);
    DqArgs a;
    a.Wd = Wd;
    a.Wq = Wq;
    a.h = h;
    a.yd = yd;
    a.words = words;
    a.pro = pro;
    a.yq = yq;
    a.epoch = tag.epoch;
    a.tag_mul = tag.mul;
    a.tag_add = tag.add;
    a.err = err;
    a.spin = attn_spin_limit();
    a.poll_xor = attn_poll_xor();
    a.units_d = (int)Wd.nb;
    a.units_q = (int)Wq.nb;
    a.wstride = sh.wstride;
    a.lds_q = (uint32_t)sh.lds_q;
    a.lds_x = (uint32_t)sh.lds_x;
    const void *k = dq_pick(Wd, sh);
    void *args[] = {&a};
    return hipLaunchKernel(k, dim3((unsigned)sh.grid), dim3(64 * sh.nwv), args, sh.lds, s);
}

}  // namespace g4
