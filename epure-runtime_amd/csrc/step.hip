// One-launch batch-1 decode step: the tuned variants (exact shapes) and the
// dispatch.  The kernel itself is in step_kernel.h; the generic variants
// (any slab-multiple shape within their maxima) are instantiated in
// step_gen_a.hip and step_gen_b.hip, so the builds run in parallel.
#include "step_kernel.h"

namespace ep {
namespace {

// Llama-3-8B, Qwen3-1.7B, Qwen3-8B and Llama-3.2-3B shapes (Qwen3-4B below); shares at 256
// workgroups: q|k|v 6 / 4 / 6 / 5 quads, o 8 / 4 / 8 / 6 (on at least half
// the grid), gate|up 14 / 6 / 12 / 8, down 4 / 2 / 4 / 3.
// Llama-3-8B: q|k|v and o whole shares in flight, gate|up 4 of 7 blocks
// issued during the attention window (5: 1.167 ms per step, 4: 1.141, 3:
// 1.163 with per-wave staging) and 1 during o, down 3 of 4 (issued during
// gate|up); Qwen3-8B the same (4 early blocks: 1.217 -> 1.170 ms).
using ModelL8B = Model<4096, 4096, 14336, 4, 3, 2, 2, 4, 6, 8, 14, 4, -1, -1, 6, 4, 4>;
using ModelQ17 = Model<2048, 2048, 6144, 2, 1, 1, 1, 1, 4, 4, 6, 2>;
using ModelQ8B = Model<4096, 4096, 12288, 4, 3, 2, 2, 4, 6, 8, 12, 4, -1, -1, 6, 4, 4>;
using ModelL3B = Model<3072, 3072, 8192, 3, 2, 2, 2, 3, 5, 6, 8, 3>;
// Qwen3-4B: hidden 2560 but 32 x 128 query columns; shares q|k|v 6, o 5,
// gate|up 10 (9.5), down 3 (2.5) quads
using ModelQ4B = Model<2560, 4096, 9728, 4, 3, 3, 2, 3, 6, 5, 10, 3>;

}  // namespace

// Which persistent variant serves the shape (0: none) and why not.
static int variant_of(const StepDesc &d)
{
    if (d.D != kD || d.levels > 16 || d.levels < 1 ||
        d.group < 128 || (d.group & (d.group - 1)) != 0 ||
        (d.scale_dtype != EP_F16 && d.scale_dtype != EP_F32) ||
        (d.cb_dtype != EP_F32 && d.cb_dtype != EP_F16) || d.Hkv < 1 ||
        d.Hq % d.Hkv != 0 || d.max_pos < 64 || d.max_pos % 64 != 0) {
        set_error(EP_DECLINE_SHAPE,
                  "decode step: head_dim %d, levels %d, group %d, scale dtype %d, cb dtype %d, "
                  "max_pos %d not served",
                  d.D, d.levels, d.group, d.scale_dtype, d.cb_dtype, d.max_pos);
        return 0;
    }
    if (d.H % d.group != 0 || d.I % d.group != 0 || (d.Hq * d.D) % d.group != 0) {
        set_error(EP_DECLINE_SHAPE, "decode step: K not a multiple of the group");
        return 0;
    }
    const int GQ = d.Hq / d.Hkv;
    auto is = [&](int H, int HQD, int I, int gq) {
        return d.H == H && d.Hq * d.D == HQD && d.I == I && GQ == gq;
    };
    if (d.scale_dtype == EP_F16) {  // the tuned variants: fp16 scales
        if (is(ModelL8B::H, ModelL8B::HQD, ModelL8B::I, ModelL8B::GQ))
            return 1;
        if (is(ModelQ17::H, ModelQ17::HQD, ModelQ17::I, ModelQ17::GQ))
            return 2;
        if (is(ModelQ8B::H, ModelQ8B::HQD, ModelQ8B::I, ModelQ8B::GQ))
            return 3;
        if (is(ModelL3B::H, ModelL3B::HQD, ModelL3B::I, ModelL3B::GQ))
            return 4;
        if (is(ModelQ4B::H, ModelQ4B::HQD, ModelQ4B::I, ModelQ4B::GQ))
            return 5;
    }
    // the generic variants: slab-multiple rows within their maxima
    const int HQD = d.Hq * d.D;
    if (GQ >= 1 && GQ <= 8 && d.H % 512 == 0 && HQD % 512 == 0 && d.I % 512 == 0 && d.H <= kGenH &&
        HQD <= kGenH && d.I <= kGenI)
        return 6;
    set_error(EP_DECLINE_SHAPE,
              "decode step: no persistent variant for hidden %d, heads %d/%d, intermediate %d "
              "(generic: hidden, heads x head_dim <= %d and intermediate <= %d, multiples of 512, "
              "GQ <= 8)",
              d.H, d.Hq, d.Hkv, d.I, kGenH, kGenI);
    return 0;
}

int decode_step_serves(const StepDesc &d) { return variant_of(d) != 0 ? EP_OK : EP_DECLINE_SHAPE; }

size_t decode_step_workspace(int H, int I, int Hq, int Hkv, int D, int max_pos)
{
    return step_ws(H, I, Hq, Hkv, D, max_pos).total;
}

int launch_decode_step(const StepDesc &d, hipStream_t stream)
{
    const int var = variant_of(d);
    if (var == 0)
        return EP_DECLINE_SHAPE;
    if (d.n_layers > 100)
        return set_error(EP_DECLINE_SHAPE, "decode step: %d layers (at most 100)", d.n_layers);
    const StepWs w = step_ws(d.H, d.I, d.Hq, d.Hkv, d.D, d.max_pos);
    if (d.ws_bytes < w.total)
        return set_error(EP_ERR_ARG, "decode step: workspace %zu < %zu bytes", d.ws_bytes, w.total);
    if (var == 6) {
        const int gq = d.Hq / d.Hkv;
        const bool sf32 = d.scale_dtype == EP_F32;
        return gq <= 4 ? launch_decode_step_gen_a(d, gq, sf32, stream)
                       : launch_decode_step_gen_b(d, gq, sf32, stream);
    }
    const StepArgs a = make_step_args(d);
    switch (var) {
    case 1:
        return launch_model<ModelL8B>(a, stream);
    case 2:
        return launch_model<ModelQ17>(a, stream);
    case 3:
        return launch_model<ModelQ8B>(a, stream);
    case 4:
        return launch_model<ModelL3B>(a, stream);
    default:
        return launch_model<ModelQ4B>(a, stream);
    }
}

size_t decode_step_layer_bytes() { return sizeof(StepLayer); }

}  // namespace ep
