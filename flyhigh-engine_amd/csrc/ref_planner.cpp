// The reference engine's conv planner, restated as host logic: candidate lists, fixed routing, the split-K
// heuristic and the dispatch words each candidate records. It runs no GPU code; tests compare its output with the
// reference's golden plans (crates/flyhigh-engine/tests/golden/*.txt) to pin the planner's choice of kernel, grid,
// K/N padding and split-K per layer.
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "common.h"
#include "fhc_conv.h"

namespace {

// candidate codes: crates/flyhigh-engine/src/ops/conv/candidates.rs:5-14
enum : uint8_t {
    CAND_DIRECT = 0,
    CAND_TC = 1,
    CAND_TILED = 2,
    CAND_TILED8 = 3,
    CAND_DIRECT64 = 4,
    CAND_TILED16 = 5,
    CAND_TILEDN8 = 6,
    CAND_TILED88 = 7,
    CAND_TILEDM32 = 8,
    CAND_TILED8P = 9,
};
const char* const kCandNames[10] = {"direct",  "tc",      "tiled",    "tiled8",   "direct64",
                                    "tiled16", "tiledn8", "tiled88",  "tiledm32", "tiled8p"};

uint32_t div_ceil(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

// candidates.rs:28-85
std::vector<uint8_t> cand_list(bool coop, uint32_t cout, uint32_t hout, uint32_t wout, bool direct_ok, bool try_all) {
    std::vector<uint8_t> cands = {CAND_DIRECT, CAND_DIRECT64, CAND_TC};
    for (uint8_t k : {CAND_TILED, CAND_TILED8, CAND_TILED16, CAND_TILEDN8, CAND_TILED88, CAND_TILEDM32, CAND_TILED8P}) {
        cands.push_back(k);
        uint32_t tm, tn;
        if (cout <= 32) {
            tm = 128;
            tn = k == CAND_TILED16 ? 16 : k == CAND_TILEDN8 ? 8 : 32;
        } else {
            tm = (k == CAND_TILED8 || k == CAND_TILED88 || k == CAND_TILED8P) ? 128 : k == CAND_TILEDM32 ? 32 : 64;
            tn = 64;
        }
        uint32_t ntiles = cout <= 32 ? div_ceil(cout, tn) : div_ceil(cout, 64);
        if (ntiles * div_ceil(hout * wout, tm) < 512)
            for (uint8_t ks : {1, 2, 4}) cands.push_back((uint8_t)(k | (ks << 4)));
    }
    std::vector<uint8_t> out;
    for (uint8_t c : cands) {
        uint8_t kid = c & 15;
        if ((kid == CAND_DIRECT || kid == CAND_DIRECT64) && !direct_ok) continue;
        if ((kid == CAND_DIRECT64 || kid == CAND_TILEDM32 || kid == CAND_TILED8P) && !try_all) continue;
        if (kid == CAND_TC && !coop) continue;
        if ((kid == CAND_TILED8 || kid == CAND_TILED88 || kid == CAND_TILEDM32 || kid == CAND_TILED8P) && cout <= 32)
            continue;
        if (kid == CAND_TILED16 && cout > 32) continue;
        if (kid == CAND_TILEDN8 && cout > 16) continue;
        out.push_back(c);
    }
    return out;
}

void emit(std::string& s, const char* pipe, uint32_t gx, uint32_t gy, uint32_t gz, uint64_t wbytes,
          const std::vector<uint32_t>& p) {
    char buf[64];
    snprintf(buf, sizeof buf, "%s (%u,%u,%u) w%llu p", pipe, gx, gy, gz, (unsigned long long)wbytes);
    s += buf;
    for (size_t i = 0; i < p.size(); i++) {
        snprintf(buf, sizeof buf, "%s%08x", i ? " " : "", p[i]);
        s += buf;
    }
    s += "\n";
}

uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

// ImplicitGemmParams as gemm_params fills it (kernels.rs:79-98)
std::vector<uint32_t> gemm_params(const fhc_ref_conv& c, uint32_t hout, uint32_t wout, uint32_t kp, uint32_t np,
                                  uint32_t cinp, uint32_t ksplit, uint32_t residual) {
    return {c.cin, c.h, c.w, hout, wout, c.stride, 1, c.cin * 9, kp, c.cout, np, hout * wout, cinp, ksplit, residual, 0};
}

// the separate residual add after a tensor-core conv (autotune.rs:135-139; elementwise.rs:8-27; step.rs:90-92)
void emit_binary(std::string& s, uint32_t c, uint32_t h, uint32_t w) {
    emit(s, "binary", div_ceil(w, 8), div_ceil(h, 8), c, 0,
         {c, h, w, c, 0, 0, 0, 0, f32_bits(1.0f), f32_bits(1.0f), 0, 0});
}

}  // namespace

extern "C" int fhc_ref_cand_list(int coop, uint32_t cout, uint32_t hout, uint32_t wout, int direct_ok, int try_all,
                                 uint8_t* out, size_t cap) {
    return fhc::guard(-1, [&]() -> int {
        std::vector<uint8_t> l = cand_list(coop != 0, cout, hout, wout, direct_ok != 0, try_all != 0);
        if (!out && cap) return fhc::fail(-1, "fhc_ref_cand_list: NULL output");
        if (l.size() > cap) return fhc::fail(-1, "fhc_ref_cand_list: %zu entries do not fit in %zu", l.size(), cap);
        for (size_t i = 0; i < l.size(); i++) out[i] = l[i];
        return (int)l.size();
    });
}

extern "C" int fhc_ref_cand_name(uint8_t code, char* buf, size_t cap) {
    return fhc::guard(-1, [&]() -> int {
        uint8_t kid = code & 15, ks = code >> 4;
        if (kid > 9) return fhc::fail(-1, "fhc_ref_cand_name: unknown kernel id %u", kid);
        std::string s = kCandNames[kid];
        if (ks) s += "/k" + std::to_string(ks);  // candidates.rs:17-24
        return fhc::write_string(s, buf, cap);
    });
}

extern "C" int fhc_ref_conv_steps(const fhc_ref_conv* cp, char* text, size_t cap) {
    return fhc::guard(-1, [&]() -> int {
        if (!cp) return fhc::fail(-1, "fhc_ref_conv_steps: NULL conv");
        const fhc_ref_conv& c = *cp;
        if (c.cin == 0 || c.cout == 0 || c.h == 0 || c.w == 0 || (c.stride != 1 && c.stride != 2))
            return fhc::fail(-1, "fhc_ref_conv_steps: bad conv %ux%u %u->%u s%u", c.w, c.h, c.cin, c.cout, c.stride);
        const uint32_t el = c.f32_mode ? 4 : 2;
        // out_size (kernels.rs:40-42)
        const uint32_t hout = (c.h + 2 - 3) / c.stride + 1, wout = (c.w + 2 - 3) / c.stride + 1, m = hout * wout;
        // fixed routing when autotune is off (autotune.rs:162-163, :191-198)
        const bool direct_ok = c.coop && c.stride == 1 && c.w % 16 == 0 && c.cout > 32;
        uint8_t cand = (uint8_t)c.cand;
        if (c.cand == 0xFF) cand = direct_ok ? CAND_DIRECT : c.coop ? CAND_TC : CAND_TILED;
        const uint8_t kid = cand & 15;
        const uint32_t ks_forced = cand >> 4;
        std::string s;
        if (kid == CAND_DIRECT || kid == CAND_DIRECT64) {
            // buildb_tap (kernels.rs:194-207), xshift3 (:226-239), conv_direct / conv_direct64 (:242-279)
            const uint32_t cinp = div_ceil(c.cin, 16) * 16, kp = 9 * cinp, np = div_ceil(c.cout, 64) * 64;
            emit(s, "xshift", div_ceil(c.w / 8, 64), c.h + 2, 3 * cinp, 0, {c.cin, cinp, c.h, c.w});
            const auto p = gemm_params(c, c.h, c.w, kp, np, cinp, 0, 0);
            if (kid == CAND_DIRECT) {
                const bool wide = c.w % 16 == 0 && m % 32 == 0;
                emit(s, wide ? "fdirect32" : "fdirect", np / 64, wide ? m / 32 : m / 16, 1, (uint64_t)kp * np * el, p);
            } else {
                emit(s, "fdirect64", np / 64, div_ceil(m, 64), 1, (uint64_t)kp * np * el, p);
            }
            if (c.residual) emit_binary(s, c.cout, hout, wout);
            return fhc::write_string(s, text, cap);
        }
        // buildb (kernels.rs:66-78)
        const uint32_t kp = div_ceil(c.cin * 9, 16) * 16;
        const uint32_t nblk = c.cout <= 32 ? 32 : 64;
        const uint32_t np = div_ceil(c.cout, nblk) * nblk;
        if (kid == CAND_TC) {
            // conv_tc (kernels.rs:100-115)
            const uint32_t mp = div_ceil(m, 16) * 16;
            emit(s, c.cout <= 32 ? "fused2" : "fused", np / nblk, mp / 16, 1, (uint64_t)kp * np * el,
                 gemm_params(c, hout, wout, kp, np, 0, 0, 0));
            if (c.residual) emit_binary(s, c.cout, hout, wout);
            return fhc::write_string(s, text, cap);
        }
        // conv_cand tiled variants (autotune.rs:142-153) -> conv_tiled_with (kernels.rs:125-191)
        uint32_t variant = 0, tn_small = 32;
        switch (kid) {
            case CAND_TILED8: variant = 1; break;
            case CAND_TILED16: tn_small = 16; break;
            case CAND_TILEDN8: tn_small = 8; break;
            case CAND_TILED88: variant = 2; break;
            case CAND_TILEDM32: variant = 3; break;
            case CAND_TILED8P: variant = 4; break;
            case CAND_TILED: break;
            default: return fhc::fail(-1, "fhc_ref_conv_steps: unknown candidate %u", cand);
        }
        const char* ker;
        uint32_t tm, tn;
        if (c.cout <= 32) {
            ker = tn_small == 8 ? "tconvn8" : tn_small == 16 ? "tconv16" : "tconv32";
            tm = 128;
            tn = tn_small;
        } else {
            switch (variant) {
                case 1: ker = "tconv8"; tm = 128; break;
                case 2: ker = "tconv88"; tm = 128; break;
                case 3: ker = "tconvm32"; tm = 32; break;
                case 4: ker = "tconv8p"; tm = 128; break;
                default: ker = "tconv"; tm = 64; break;
            }
            tn = 64;
        }
        const uint32_t gx = c.cout <= 32 ? div_ceil(c.cout, tn) : np / tn, gy = div_ceil(m, tm);
        const uint32_t kt_count = kp / 16, kt1 = kt_count > 1 ? kt_count : 1;
        uint32_t ksplit;
        if (ks_forced > 0)
            ksplit = ks_forced < kt1 ? ks_forced : kt1;
        else if (gx * gy >= 512)
            ksplit = 1;
        else {
            ksplit = div_ceil(512, gx * gy);
            if (ksplit > 8) ksplit = 8;
            if (ksplit > kt1) ksplit = kt1;
        }
        if (c.ksplit_env) ksplit = c.ksplit_env < kt1 ? c.ksplit_env : kt1;  // FH_KSPLIT (kernels.rs:164-166)
        while (ksplit > 1 && (uint64_t)(uint32_t)(ksplit * c.cout * m) * 4 > (32u << 20)) ksplit--;
        const uint64_t wb = (uint64_t)kp * np * el;
        if (ksplit <= 1) {
            emit(s, ker, gx, gy, 1, wb, gemm_params(c, hout, wout, kp, np, 0, ksplit, c.residual ? 1 : 0));
        } else {
            emit(s, ker, gx, gy, ksplit, wb, gemm_params(c, hout, wout, kp, np, 0, ksplit, 0));
            emit(s, "skreduce", div_ceil(c.cout * m / 4, 256), 1, 1, 0, {c.cout, m, ksplit, c.residual ? 1u : 0u});
        }
        return fhc::write_string(s, text, cap);
    });
}
