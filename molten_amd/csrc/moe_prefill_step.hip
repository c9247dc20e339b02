// moe_prefill_step.hip -- the whole prefill MoE block in one call
// (src/lfm.rs:847-965 moe_prefill), on a caller-provided workspace.
//
// Sequence (five launches and the combine): router logits (expert rows held
// in the LDS, tokens streamed) -> per-token top-k with per-block expert
// histograms -> counts, offsets, block-map offsets, the stable scatter and
// the block maps, also in the GEMMs' launch order (every workgroup sums the
// histograms) -> grouped gate/up
// GEMM with the ids_sorted row gather and the SwiGLU epilogue fused ->
// grouped down GEMM -> weighted combine.  Compared with the reference's sequence this drops the
// materialised gathered rows and the separate gate/up outputs (two 4-byte
// round trips per routed element); the values are the same.
#include <algorithm>

#include "mh_device.hpp"
#include "mh_host.hpp"

namespace {

constexpr uint32_t kBM = 512;      // row tile of both grouped GEMMs (segment kernels)
constexpr uint32_t kGuBN = 128;    // gate/up tile width (fused SwiGLU)
constexpr uint32_t kDnBN = 256;    // down tile width

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

struct Layout {
    size_t off[MH_PREFILL_WS_REGIONS];
    size_t total;
    uint32_t max_gu, max_dn;
    bool ordered;              // launch-ordered maps (the map's rows fit the scatter's ranking)
    uint32_t grid_gu, grid_dn;  // their entries: the GEMMs' workgroups
};

Layout layout_for(uint32_t m, uint32_t e, uint32_t topk, uint32_t d_model, uint32_t n_inter) {
    const size_t s = static_cast<size_t>(m) * topk;
    const uint32_t m_tiles = static_cast<uint32_t>((s + kBM - 1) / kBM) + e;
    Layout l{};
    l.max_gu = m_tiles * (n_inter / kGuBN);
    l.max_dn = m_tiles * (d_model / kDnBN);
    l.ordered = m_tiles <= mh::kMaxOrderedRows;
    l.grid_gu = mh::map_grid(l.max_gu, n_inter / kGuBN);
    l.grid_dn = mh::map_grid(l.max_dn, d_model / kDnBN);
    const size_t sizes[MH_PREFILL_WS_REGIONS] = {
        static_cast<size_t>(m) * e * 4,  // logits f32 [m, e]
        s * 4,                           // ids u32 [m, topk]
        s * 2,                           // gw bf16 [m, topk]
        static_cast<size_t>(e) * 4,      // counts
        static_cast<size_t>(e) * 4,      // offsets
        s * 4,                           // ids_sorted
        s * 4,                           // slotpos
        static_cast<size_t>(e) * 4,      // gate/up block offsets
        static_cast<size_t>(e) * 4,      // down block offsets
        static_cast<size_t>(l.max_gu) * 16,  // gate/up block map
        static_cast<size_t>(l.max_dn) * 16,  // down block map
        s * n_inter * 2,                 // act bf16 [s, n_inter]
        std::max(s * d_model * 2,        // ed bf16 [s, d_model]; before the down GEMM, the
                                         // routing's block histograms and expert totals
                 (static_cast<size_t>((m + mh::kPrefillRouteBlock - 1) / mh::kPrefillRouteBlock) + 1) * e * 4),
        l.ordered ? static_cast<size_t>(l.grid_gu) * 16 : 0,  // gate/up map in launch order
        l.ordered ? static_cast<size_t>(l.grid_dn) * 16 : 0,  // down map in launch order
    };
    size_t at = 0;
    for (int i = 0; i < MH_PREFILL_WS_REGIONS; ++i) {
        l.off[i] = at;
        at = align256(at + sizes[i]);
    }
    l.total = at;
    return l;
}

}  // namespace

extern "C" {

size_t mh_moe_prefill_workspace(uint32_t m, uint32_t n_experts, uint32_t topk, uint32_t d_model,
                                uint32_t n_inter, size_t* offsets) {
    const Layout l = layout_for(m, n_experts, topk, d_model, n_inter);
    if (offsets) {
        for (int i = 0; i < MH_PREFILL_WS_REGIONS; ++i) offsets[i] = l.off[i];
    }
    return l.total;
}

}  // extern "C"

namespace {

// mh_moe_prefill, and with stamps != null its measured form (the two grouped
// GEMMs with workgroup stamps).
int prefill(const char* op, const void* router, int router_dtype, const float* bias, int mode, float eps,
            const mh_quant_weights* gate, const mh_quant_weights* up, const mh_quant_weights* down,
            uint32_t n_experts, uint32_t topk, const uint16_t* x, uint32_t m, uint16_t* out, void* workspace,
            size_t workspace_bytes, mh_stream_t stream, uint64_t* stamps) {
    MH_ENSURE(gate && up && down && x && out && workspace && router, MH_ERR_INVALID,
              "%s: NULL argument", op);
    MH_ENSURE(m > 0, MH_ERR_INVALID, "%s: no tokens", op);
    MH_ENSURE(n_experts > 0 && n_experts <= 256 && gate->out_features % n_experts == 0 &&
                  down->out_features % n_experts == 0,
              MH_ERR_INVALID, "%s: stacked rows not divisible by %u experts", op, n_experts);
    const uint32_t n_inter = gate->out_features / n_experts;
    const uint32_t d_model = down->out_features / n_experts;
    MH_ENSURE(gate->in_features == d_model && up->in_features == d_model &&
                  up->out_features == gate->out_features && down->in_features == n_inter,
              MH_ERR_INVALID, "%s: expert shapes do not chain", op);
    MH_ENSURE(n_inter % kGuBN == 0 && d_model % kDnBN == 0, MH_ERR_UNSUPPORTED,
              "%s: n_inter %% %u or d_model %% %u != 0", op, kGuBN, kDnBN);
    MH_ENSURE(topk >= 1 && topk <= 8, MH_ERR_INVALID, "%s: topk %u", op, topk);
    MH_ENSURE(mh::aligned(workspace, 256) && mh::aligned(x, 16) && mh::aligned(out, 16),
              MH_ERR_ALIGN, "%s: workspace must be 256-byte aligned, x/out 16-byte aligned", op);
    const Layout l = layout_for(m, n_experts, topk, d_model, n_inter);
    MH_ENSURE(workspace_bytes >= l.total, MH_ERR_INVALID,
              "%s: workspace holds %zu bytes, needs %zu", op, workspace_bytes, l.total);
    for (const mh_quant_weights* w : {gate, up, down}) {
        MH_TRY(mh::check_quant(w, op));
        MH_ENSURE(w->bits == 4 && w->group_size == 64, MH_ERR_UNSUPPORTED,
                  "%s: experts must be 4-bit group 64", op);
    }

    char* ws = static_cast<char*>(workspace);
    auto at = [&](int region) { return ws + l.off[region]; };
    float* logits = reinterpret_cast<float*>(at(MH_PREFILL_WS_LOGITS));
    uint32_t* ids = reinterpret_cast<uint32_t*>(at(MH_PREFILL_WS_IDS));
    uint16_t* gw = reinterpret_cast<uint16_t*>(at(MH_PREFILL_WS_GW));
    uint32_t* counts = reinterpret_cast<uint32_t*>(at(MH_PREFILL_WS_COUNTS));
    uint32_t* offsets = reinterpret_cast<uint32_t*>(at(MH_PREFILL_WS_OFFSETS));
    uint32_t* ids_sorted = reinterpret_cast<uint32_t*>(at(MH_PREFILL_WS_IDS_SORTED));
    uint32_t* slotpos = reinterpret_cast<uint32_t*>(at(MH_PREFILL_WS_SLOTPOS));
    uint32_t* gu_off = reinterpret_cast<uint32_t*>(at(MH_PREFILL_WS_GU_OFF));
    uint32_t* dn_off = reinterpret_cast<uint32_t*>(at(MH_PREFILL_WS_DN_OFF));
    uint32_t* gu_map = reinterpret_cast<uint32_t*>(at(MH_PREFILL_WS_GU_MAP));
    uint32_t* dn_map = reinterpret_cast<uint32_t*>(at(MH_PREFILL_WS_DN_MAP));
    uint16_t* act = reinterpret_cast<uint16_t*>(at(MH_PREFILL_WS_ACT));
    uint16_t* ed = reinterpret_cast<uint16_t*>(at(MH_PREFILL_WS_ED));
    uint32_t* gu_ord = l.ordered ? reinterpret_cast<uint32_t*>(at(MH_PREFILL_WS_GU_ORD)) : nullptr;
    uint32_t* dn_ord = l.ordered ? reinterpret_cast<uint32_t*>(at(MH_PREFILL_WS_DN_ORD)) : nullptr;
    const uint32_t s = m * topk;

    // the block histograms of the routing live in the down GEMM's output
    // region until that GEMM runs
    // a bf16 router: logits and top-k in one launch on the matrix cores
    // (moe_route_mma.hip; the routing exact), else the chunk-order logits of
    // every expert, then the top-k
    const bool mma = mh::route_mma_fits(router, router_dtype, x, n_experts, d_model, topk);
    if (mma) {
        MH_ENSURE(mode == MH_ROUTE_SIGMOID_BIAS || mode == MH_ROUTE_SOFTMAX, MH_ERR_INVALID, "%s: mode %d", op,
                  mode);
        MH_TRY(mh::route_mma(x, static_cast<const uint16_t*>(router), bias, mode, eps, m, n_experts, d_model, topk,
                             logits, ids, gw, reinterpret_cast<uint32_t*>(ed), mh::as_stream(stream)));
    } else {
        MH_TRY(mh::router_prefill_logits(x, router, router_dtype, logits, m, d_model, n_experts, stream));
    }
    MH_TRY(mh::moe_route_sort_maps(logits, bias, mode, eps, m, n_experts, topk, ids, gw,
                                   reinterpret_cast<uint32_t*>(ed), counts, offsets, gu_off, dn_off,
                                   ids_sorted, slotpos, gu_map, l.max_gu, dn_map, l.max_dn, kBM, kGuBN,
                                   kDnBN, n_inter, d_model, stream, mma, gu_ord, dn_ord));
    if (l.ordered || stamps != nullptr) {
        // the segment kernels: on the launch-ordered maps (each workgroup reads
        // its entry, no ranking), and / or stamped
        const hipStream_t hs = mh::as_stream(stream);
        MH_TRY(mh::gemm_gu_act_seg(x, ids_sorted, m, gate, up, act, l.ordered ? gu_ord : gu_map,
                                   l.ordered ? l.grid_gu : l.max_gu, s, n_inter, kBM, kGuBN, l.ordered, stamps, hs));
        MH_TRY(mh::gemm_grouped_seg(act, down, ed, l.ordered ? dn_ord : dn_map, l.ordered ? l.grid_dn : l.max_dn, s,
                                    d_model, kBM, kDnBN, l.ordered,
                                    stamps != nullptr ? stamps + static_cast<size_t>(MH_PREFILL_STAMP_WGS) *
                                                                     MH_PREFILL_STAMPS
                                                      : nullptr,
                                    hs));
    } else {
        MH_TRY(mh_gemm_q4_grouped_gu_act(x, ids_sorted, m, gate, up, act, gu_map, l.max_gu, s, n_inter,
                                         kBM, kGuBN, stream));
        MH_TRY(mh_gemm_q4_grouped(act, down, ed, dn_map, l.max_dn, s, d_model, kBM, kDnBN, stream));
    }
    return mh_moe_combine_rows(ed, slotpos, gw, out, m, d_model, topk, stream);
}

}  // namespace

extern "C" {

int mh_moe_prefill(const void* router, int router_dtype, const float* bias, int mode, float eps,
                   const mh_quant_weights* gate, const mh_quant_weights* up,
                   const mh_quant_weights* down, uint32_t n_experts, uint32_t topk,
                   const uint16_t* x, uint32_t m, uint16_t* out, void* workspace,
                   size_t workspace_bytes, mh_stream_t stream) {
    return prefill("mh_moe_prefill", router, router_dtype, bias, mode, eps, gate, up, down, n_experts, topk, x, m,
                   out, workspace, workspace_bytes, stream, nullptr);
}

int mh_moe_prefill_stamped(const void* router, int router_dtype, const float* bias, int mode, float eps,
                           const mh_quant_weights* gate, const mh_quant_weights* up,
                           const mh_quant_weights* down, uint32_t n_experts, uint32_t topk,
                           const uint16_t* x, uint32_t m, uint16_t* out, void* workspace,
                           size_t workspace_bytes, uint64_t* stamps, mh_stream_t stream) {
    const char* op = "mh_moe_prefill_stamped";
    MH_ENSURE(stamps != nullptr && mh::aligned(stamps, 8), MH_ERR_INVALID, "%s: stamps NULL or not 8-byte aligned",
              op);
    return prefill(op, router, router_dtype, bias, mode, eps, gate, up, down, n_experts, topk, x, m, out, workspace,
                   workspace_bytes, stream, stamps);
}

}  // extern "C"
