// CPU check of the launch plans (no GPU call is made).  For model shapes of
// the BASELINE configs and others, every row count of a session, decode steps
// and prefill / head calls: each decode-shape GEMM launch the batched engine
// plans uses an instantiated (wavefronts, k-steps) pair, at most 4 row tiles
// per workgroup, and split-K partials and counters that fit what the engine
// allocates for the model (engine_part_need, CNT_GEMM); the persistent
// kernel's role split is valid for every grid of 4 to 512 workgroups; the
// decode attention's wavefronts, key splits and speculative loads at the
// decode shapes.
// Prints "plans ok" and exits 0, or names the first failing case.
#include <cstdio>
#include <cstdlib>

#include "decode_kernel.h"
#include "engine_plan.h"

using namespace dnnhip;

static int fails = 0;
#define CHECK(cond, ...)                        \
    do {                                        \
        if (!(cond)) {                          \
            if (fails++ < 10) {                 \
                std::printf("FAIL: " __VA_ARGS__); \
                std::printf("\n");              \
            }                                   \
        }                                       \
    } while (0)

static bool in(const int *a, int n, int v) {
    for (int i = 0; i < n; i++)
        if (a[i] == v) return true;
    return false;
}

static int round_to(int v, int a) { return (v + a - 1) / a * a; }

static void check_gemm(const char *what, int N, int K, int M, bool norm, int mt_max, size_t part_cap, int D) {
    const int ntn = (N + 15) / 16, nks = K / 16, tiles_m = (M + 15) / 16;
    const int ks = pick_ks(ntn, K, M, norm, mt_max);
    CHECK(ks >= 1, "%s D=%d M=%d: no split fits", what, D, M);
    if (ks < 1) return;
    const int kw = decode_kw(nks, ks);
    CHECK(nks % (kw * ks) == 0, "%s D=%d M=%d: K/16=%d over %d x %d", what, D, M, nks, kw, ks);
    const int kpw = nks / (kw * ks);
    const bool inst = kw == 8 ? in(GEMM_KPW_KW8, sizeof GEMM_KPW_KW8 / sizeof(int), kpw)
                              : in(GEMM_KPW_KW4, sizeof GEMM_KPW_KW4 / sizeof(int), kpw);
    CHECK(inst, "%s D=%d M=%d: %d wavefronts x %d k-steps not instantiated", what, D, M, kw, kpw);
    int mt = tiles_m;
    if (mt_max > 0 && mt > mt_max) mt = mt_max;
    CHECK(mt >= 1 && mt <= 4, "%s D=%d M=%d: %d row tiles per workgroup", what, D, M, mt);
    const int groups = (tiles_m + mt - 1) / mt;
    if (ks > 1) {
        const size_t need = (size_t)ks * M * N + (size_t)ntn * ks * M;
        CHECK(need <= part_cap, "%s D=%d M=%d: %zu partial pairs > %zu", what, D, M, need, part_cap);
        CHECK((size_t)groups * ntn <= (size_t)CNT_GEMM, "%s D=%d M=%d: %d counters > %d", what, D, M, groups * ntn,
              CNT_GEMM);
    }
}

static void check_model(int V, int D, int F) {
    const int ldD = round_to(D, LDALIGN), ldF = round_to(F, LDALIGN);
    const size_t cap = engine_part_need(D, F, V, ldD, ldF);
    for (int M = 1; M <= PLAN_MAX_ROWS; M++)
        for (int hd = 0; hd < 2; hd++) {
            const MtPlan p = mt_plan(M, hd != 0);
            check_gemm("qkv", 3 * D, ldD, M, true, p.qkv, cap, D);
            check_gemm("out_proj", D, ldD, M, false, p.out, cap, D);
            check_gemm("gate/up", 2 * F, ldD, M, true, p.gu, cap, D);
            check_gemm("down", D, ldF, M, false, p.down, cap, D);
            check_gemm("lm_head", V, ldD, M, true, p.head, cap, D);
        }
}

static void check_roles(int D, int F) {
    const int ldD = round_to(D, LDALIGN), ldF = round_to(F, LDALIGN);
    const int recs[] = {1, 4, 12, 24, 48, 96};
    for (int nb : {1, 2, 4, 8})
        for (int G = 4; G <= 512; G++)
            for (int r : recs) {
                Roles ro{};
                const bool ok = plan_roles(G, D, F, ldD, ldF, r, ro, hold_rounds(nb, ldD / LDALIGN));
                CHECK(ok, "roles G=%d D=%d records=%d: no split", G, D, r);
                if (!ok) continue;
                CHECK(ro.n_ac >= 1 && ro.n_d >= 1 && ro.n_e >= 1 && ro.n_ac + ro.n_d + ro.n_e <= G - 1,
                      "roles G=%d D=%d records=%d: %d/%d/%d", G, D, r, ro.n_ac, ro.n_d, ro.n_e);
            }
}

// the decode attention's wavefronts and key splits at the BASELINE decode
// shapes (12 heads; a sweep of 1-6 splits found these best)
static void check_splits() {
    CHECK(attn_waves(8, 12) == 8 && attn_waves(11, 12) == 4 && attn_waves(32, 12) == 4, "wavefronts per workgroup");
    CHECK(attn_splits_for(0, 8, 12, 1088) == 2, "C4: 8 rows x 12 heads at 1088 keys: two splits");
    CHECK(attn_splits_for(0, 8, 12, 560) == 1, "C2 at 8 rows, 560 keys: one split");
    CHECK(attn_splits_for(0, 32, 12, 320) == 1, "C3: 384 (row, head) pairs fill the chip: one split");
    CHECK(attn_splits_for(0, 64, 8, 215) == 1, "C5: one split");
    CHECK(attn_splits_for(0, 1, 12, 1 << 20) == 8, "at most eight splits");
    CHECK(attn_splits_for(0, 1, 12, 1024) == 1 && attn_splits_for(0, 1, 12, 1025) == 2,
          "one split up to 16 chunks of 64 keys (8 wavefronts x 2), two past it");
    CHECK(attn_splits_for(3, 32, 12, 320) == 3 && attn_splits_for(12, 8, 12, 64) == 8, "override, at most eight");
}

// the decode attention's speculative first-chunk loads at the BASELINE
// decode shapes (12 heads; the counts the engine measured best or within noise)
static void check_spec() {
    int pos[64];
    for (int b = 0; b < 8; b++) pos[b] = 1024 + b % 64;
    CHECK(attn_spec(8, 2, 8, 64, pos) == 8, "C4: all eight wavefronts speculative");
    for (int b = 0; b < 8; b++) pos[b] = 48;
    CHECK(attn_spec(8, 1, 8, 512, pos) == 4, "C2 at 8 rows from position 48: four (keys >= 256 in 59%%)");
    for (int b = 0; b < 32; b++) pos[b] = 16 + (48 * b) / 31;
    CHECK(attn_spec(4, 1, 32, 256, pos) == 2, "C3: two (keys >= 128 in about 66%%)");
    for (int b = 0; b < 64; b++) pos[b] = 196 + b % 4;
    CHECK(attn_spec(4, 1, 64, 16, pos) == 4, "C5: all four (every history past 192 keys)");
    pos[0] = 0;
    CHECK(attn_spec(4, 1, 1, 1, pos) == 1, "one new row: one");
    CHECK(attn_spec(8, 1, 1, 1, pos) == 4, "one new row, eight wavefronts: four");
    // the 3/4 threshold, exactly: a history of S = pos + t + 1 > 64 keys at
    // 3 of 4 steps (pos 63: t = 1..3) -> speculative; at 2 of 4 (pos 62) not
    pos[0] = 63;
    CHECK(attn_spec(4, 1, 1, 4, pos) == 2, "3 of 4 steps past 64 keys: two");
    pos[0] = 62;
    CHECK(attn_spec(4, 1, 1, 4, pos) == 1, "2 of 4 steps past 64 keys: one");
    // two key splits: wavefront w's first chunk starts at key 128 w
    pos[0] = 600;
    CHECK(attn_spec(8, 2, 1, 1, pos) == 5, "two splits, 601 keys: five (key 640 is past the history)");
    setenv("DNN_HIP_ATT_SPEC", "9", 1);
    CHECK(attn_spec(4, 1, 1, 4, pos) == 4, "override clamped to the wavefronts");
    unsetenv("DNN_HIP_ATT_SPEC");
}

int main() {
    unsetenv("DNN_HIP_ATT_SPEC");
    check_splits();
    check_spec();
    // (V, D, F): C1, C2-C4, C5, and other engine shapes (D = 64 * heads <= 768, F <= 2048)
    const int shapes[][3] = {{128, 256, 683}, {8192, 768, 2048}, {1024, 512, 1024}, {512, 256, 683},
                             {4096, 384, 1024}, {32000, 640, 1708}, {50257, 768, 2048}, {256, 128, 384},
                             {1000, 64, 256}, {65535, 768, 2048}};
    for (const auto &s : shapes) check_model(s[0], s[1], s[2]);
    // the tests' non-default row tiles
    setenv("DNN_HIP_QKV_MT", "2", 1);
    setenv("DNN_HIP_GU_MT", "2", 1);
    setenv("DNN_HIP_DOWN_MT", "0", 1);
    setenv("DNN_HIP_HEAD_MT", "1", 1);
    for (const auto &s : shapes) check_model(s[0], s[1], s[2]);
    for (const auto &s : shapes) check_roles(s[1], s[2]);
    if (fails) {
        std::printf("%d plan checks failed\n", fails);
        return 1;
    }
    std::printf("plans ok\n");
    return 0;
}
