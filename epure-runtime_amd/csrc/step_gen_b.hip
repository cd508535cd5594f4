// Generic variants of the one-launch decode step (step_kernel.h) for
// GQ = Hq / Hkv in 5..8: H and Hq * D up to 4096 and I up to 16384
// (multiples of 512), the launch's own shape read from its arguments, with
// fp16 or f32 (make_trainable) group scales.  The GEMV geometry is that of
// the maxima, tuned like the Llama-3-8B variant; smaller shapes leave some
// slabs and row quads idle.
#include "step_kernel.h"

namespace ep {
namespace {

// q|k|v share: (Hq D + 2 Hkv D) / 4 rows' quads over 256 workgroups
template <int GQ, bool SF32>
using ModelGen = Model<kGenH, kGenH, kGenI, GQ, 3, 2, 2, 4, (kGenH + 2 * kGenH / GQ + 1023) / 1024, 8, kGenI / 1024,
                       4, -1, -1, 6, 4, 4, true, SF32>;

template <int GQ>
int launch_gq(const StepArgs &a, bool sf32, hipStream_t stream)
{
    return sf32 ? launch_model<ModelGen<GQ, true>>(a, stream) : launch_model<ModelGen<GQ, false>>(a, stream);
}

}  // namespace

int launch_decode_step_gen_b(const StepDesc &d, int gq, bool sf32, hipStream_t stream)
{
    const StepArgs a = make_step_args(d);
    switch (gq) {
    case 5:
        return launch_gq<5>(a, sf32, stream);
    case 6:
        return launch_gq<6>(a, sf32, stream);
    case 7:
        return launch_gq<7>(a, sf32, stream);
    case 8:
        return launch_gq<8>(a, sf32, stream);
    default:
        return set_error(EP_DECLINE_SHAPE, "decode step: GQ %d not in this unit", gq);
    }
}

}  // namespace ep
