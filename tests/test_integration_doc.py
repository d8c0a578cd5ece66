"""The C++ shim that keeps the reference's qw::gpu names (shown for
maintainers in the integration guide) compiles against include/qw/q4ops.h
when called with the engine's own buffer types,
and the Python ctypes stub there declares the argument count the C-ABI has."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GUIDE = os.path.join(ROOT, "INTEGRATION.md")


def blocks(lang):
    return re.findall(r"```" + re.escape(lang) + r"\n(.*?)```", open(GUIDE).read(), flags=re.S)


# Calls of every shim wrapper with the engine's own buffer types: the
# decode rows of Rank::Batch and the prefill rows of PrefillBuf
# (src/engine/rank.hpp:51-71,163-170 of the reference): fp16 rows and
# intermediates are uint16_t *, fp32 rows float *, indices int32_t *, and the
# reference's own argument kinds (bool accumulate / f16_out, int rpg, a
# rocblas_handle). A wrapper that took another buffer type (an fp32 yp, a
# bf16 flag) fails to compile here.
ENGINE_CALLS = r"""
struct Batch {  // Rank::Batch's fields used here; top_e, active, n_active are the integration's additions
    float *X, *hc_send, *router, *tok_w, *shp, *sh_out, *out_moe, *proj, *logits;
    uint16_t *y, *bin, *moe_h, *yp, *sh_h;
    int32_t *counts, *offsets, *tok_slot, *pair_tok, *top_e, *active, *n_active;
};
struct PrefillBuf {  // PrefillBuf's fields used here; top_e, active, n_active, tile_e, tile_m0, n_tiles added
    float *logits, *tok_w, *d;
    uint16_t *xn, *bin, *part16, *moe_h, *yp, *sh_h, *sh_out;
    int32_t *counts, *offsets, *tok_slot, *pair_tok, *top_e, *active, *n_active, *tile_e, *tile_m0, *n_tiles;
};
void engine_calls(Batch &b, PrefillBuf &p, rocblas_handle blas, hipStream_t s, const uint16_t *w16,
                  const qw::gpu::W16t &sh_gu, const qw::gpu::W16t &sh_down, const qw::gpu::Q4 &wq,
                  const qw::gpu::Q4 &g, const qw::gpu::Q4 &u, const qw::gpu::Q4 &d, const qw::gpu::Q8t &w8,
                  const qw::gpu::MoeShape &sh, const uint16_t *router_w, void *ws, size_t ws_bytes) {
    const int M = 4, T = 4096, HC = 4, SH = 1024, HC_DOWN = 324, HC_SEND = 1300;
    bool accumulate = false, f16_out = true;
    int rpg = HC_DOWN;
    // decode.hip:55-59: the hyper-connection down projection, rows grouped by stream
    qw::gpu::gemv_rows(w16, b.y, HC * SH, b.hc_send + HC, HC_SEND, HC * HC_DOWN, SH, M, rpg, accumulate, s);
    qw::gpu::gemv_rows_i8(w8, b.y, HC * SH, b.hc_send + HC, HC_SEND, M, HC_DOWN, false, s);
    qw::gpu::gemv_rows(wq, b.bin, sh.H, b.proj, wq.N, M, 0, accumulate, s);
    // decode.hip:99-111: router, route, experts, combine, shared expert
    qw::gpu::moe_route_B(b.router, M, sh,
                         qw::gpu::MoeRoute{b.counts, b.offsets, b.tok_slot, b.pair_tok, b.tok_w, b.top_e, b.active,
                                           b.n_active, nullptr, nullptr, nullptr},
                         s);
    const qw::gpu::MoeRoute rb{b.counts, b.offsets, b.tok_slot, b.pair_tok, b.tok_w, b.top_e, b.active, b.n_active,
                               nullptr, nullptr, nullptr};
    qw::gpu::moe_experts_P(g, u, d, sh, rb, b.bin, M, b.moe_h, b.yp, s);
    qw::gpu::gemv_rows(sh_gu, b.bin, sh.H, b.sh_out, sh_gu.N, M, 0, false, s);
    qw::gpu::swiglu_T(b.sh_out, sh_gu.N, sh_down.K, M, b.sh_h, s);
    qw::gpu::gemv_rows(sh_down, b.sh_h, sh_down.K, b.proj, sh.H, M, 0, false, s);
    qw::gpu::swiglu_T_gemv_rows(sh_down, b.sh_out, sh_gu.N, b.proj, sh.H, M, false, s);
    qw::gpu::moe_combine_B(b.yp, b.tok_slot, b.tok_w, b.proj, M, sh, b.out_moe, s);
    qw::gpu::moe_block_B(router_w, b.bin, M, g, u, d, sh, b.proj, b.out_moe, b.logits, b.top_e, b.tok_w, b.tok_slot,
                         b.moe_h, b.yp, ws, ws_bytes, s);
    qw::gpu::moe_block_shared_B(router_w, b.bin, M, g, u, d, sh, sh_gu, sh_down, b.shp, b.sh_out, b.out_moe,
                                b.logits, b.top_e, b.tok_w, b.tok_slot, b.moe_h, b.yp, ws, ws_bytes, s);
    // prefill.hip:324-339: router GEMM (fp32 out), experts, shared expert (fp16 out), combine
    qw::gpu::gemm(blas, wq, p.bin, sh.H, T, p.logits, sh.E, false);
    qw::gpu::gemm(blas, wq, p.bin, sh.H, T, p.part16, wq.N, f16_out);
    const qw::gpu::MoeRoute rp{p.counts, p.offsets, p.tok_slot, p.pair_tok, p.tok_w, p.top_e, p.active, p.n_active,
                               p.tile_e, p.tile_m0, p.n_tiles};
    qw::gpu::moe_route_T(p.logits, T, sh, rp, s);
    qw::gpu::moe_experts_T(g, u, d, sh, rp, p.bin, T, p.moe_h, p.yp, s);
    qw::gpu::moe_experts_T(g, u, d, sh, rp, p.bin, T, p.moe_h, p.yp, s, ws, ws_bytes);
    qw::gpu::moe_combine_T(p.yp, p.tok_slot, p.tok_w, p.sh_out, T, sh, p.part16, s);
}
int main() { return 0; }
"""


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not on PATH")
def test_shim_compiles(tmp_path):
    shim = [b for b in blocks("c++") if "#pragma once" in b and "namespace qw::gpu" in b]
    assert len(shim) == 1
    src = tmp_path / "shim_check.hip"
    src.write_text(shim[0].replace("#pragma once\n", "") + ENGINE_CALLS)
    r = subprocess.run(["hipcc", "--offload-arch=gfx950", "-std=c++17", "-fsyntax-only",
                        "-I", os.path.join(ROOT, "include"), str(src)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]


def test_ctypes_stub_arity_matches_header():
    stub = [b for b in blocks("python") if "argtypes" in b][0]
    n_stub = len(re.search(r"qw_q4_gemv\.argtypes = \[(.*?)\]", stub).group(1).split(","))
    header = open(os.path.join(ROOT, "include", "qw", "q4ops.h")).read()
    decl = re.search(r"int qw_q4_gemv\((.*?)\);", header, flags=re.S).group(1)
    assert n_stub == len(decl.split(","))
