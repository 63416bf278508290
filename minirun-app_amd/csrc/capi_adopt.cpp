// Adopted affine weights: AffineWeights.adopting (MLXBridge/AffineWeights.swift:
// 159-198) over the C-ABI.  Three caller buffers, each with its finalizer, and a
// reference count shared by the holders of the weight (copies of the Swift
// value); releases may come from any thread (BufferPool.swift:45-90).  The
// last release runs every finalizer exactly once: behind the GPU work of the
// stream it names (a host function on that stream; NULL is the default
// stream, as everywhere in the ABI), or on the releasing thread through
// mr_adopted_affine_release_now when no GPU work reads the weight any more.
// Live handles are kept in a registry, so a call with a released handle is
// rejected without touching freed memory.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <new>
#include <unordered_set>

#include "../../include/minirun_hip.h"
#include "capi_util.hpp"

struct mr_adopted_affine {
    int32_t refs;  // guarded by the registry lock
    mr_affine_weight w;
    mr_finalizer fin[3];
    void* ctx[3];
};

namespace {

using mrc::fail;
using mrc::hip_fail;

std::mutex g_mu;
std::unordered_set<const mr_adopted_affine*>& registry() {
    static std::unordered_set<const mr_adopted_affine*> live;  // never destroyed before late releases
    return live;
}

void run_finalizers(mr_finalizer const* fin, void* const* ctx) {
    for (int i = 0; i < 3; ++i)
        if (fin[i]) fin[i](ctx[i]);
}

// The last holder is gone and the stream has passed every read.
void finish(void* p) {
    mr_adopted_affine* a = static_cast<mr_adopted_affine*>(p);
    run_finalizers(a->fin, a->ctx);
    delete a;
}

// Drops one reference under the registry lock.  Returns MR_OK and sets
// *last when this was the last one (the handle has then left the registry).
mr_status drop_ref(mr_adopted_affine* a, const char* who, bool* last) {
    std::lock_guard<std::mutex> lock(g_mu);
    if (!a || !registry().count(a)) return fail(MR_INVALID_ARGUMENT, "%s: not a live adopted weight", who);
    *last = --a->refs == 0;
    if (*last) registry().erase(a);
    return MR_OK;
}

}  // namespace

extern "C" {

mr_status mr_affine_adopt(void* packed, void* scales, void* biases, mr_dtype scale_dtype, int64_t experts,
                          int64_t out_features, int64_t in_features, int32_t group, int32_t bits,
                          mr_finalizer packed_finalizer, void* packed_context, mr_finalizer scales_finalizer,
                          void* scales_context, mr_finalizer biases_finalizer, void* biases_context,
                          mr_adopted_affine** out) {
    mr_finalizer fin[3] = {packed_finalizer, scales_finalizer, biases_finalizer};
    void* ctx[3] = {packed_context, scales_context, biases_context};
    // the buffers belong to the weight from here on: a failure drops it, and
    // dropping it runs the finalizers (the reference's arrays own the pointers
    // before its validation runs, AffineWeights.swift:166-170)
    auto drop = [&](mr_status st) {
        run_finalizers(fin, ctx);
        return st;
    };
    if (out) *out = nullptr;
    if (!out) return drop(fail(MR_INVALID_ARGUMENT, "mr_affine_adopt: out is NULL"));
    // the shapes the reference builds (AffineWeights.swift:185-190), checked
    // as AffineWeights.init checks them
    const int64_t words = bits > 0 ? in_features * bits / 32 : 0;
    const int64_t groups = group > 0 ? in_features / group : 0;
    const int32_t rank = experts != 0 ? 3 : 2;
    const int64_t ps[3] = {experts, out_features, words}, ss[3] = {experts, out_features, groups};
    const int64_t* pshape = rank == 3 ? ps : ps + 1;
    const int64_t* sshape = rank == 3 ? ss : ss + 1;
    int64_t ex = 0, of = 0, inf = 0;
    const mr_status st = mr_affine_validate(MR_U32, rank, pshape, scale_dtype, rank, sshape, scale_dtype, rank,
                                            sshape, group, bits, &ex, &of, &inf);
    if (st != MR_OK) return drop(st);
    if (!packed || !scales || !biases)
        return drop(fail(MR_INVALID_ARGUMENT, "mr_affine_adopt: packed, scales and biases must be non-NULL"));
    mr_adopted_affine* a = new (std::nothrow) mr_adopted_affine;
    if (!a) return drop(fail(MR_INVALID_ARGUMENT, "mr_affine_adopt: out of host memory"));
    a->refs = 1;
    a->w.packed = static_cast<const uint32_t*>(packed);
    a->w.scales = scales;
    a->w.biases = biases;
    a->w.scale_dtype = scale_dtype;
    a->w.out_features = of;
    a->w.in_features = inf;
    a->w.group = group;
    a->w.bits = bits;
    for (int i = 0; i < 3; ++i) {
        a->fin[i] = fin[i];
        a->ctx[i] = ctx[i];
    }
    {
        std::lock_guard<std::mutex> lock(g_mu);
        registry().insert(a);
    }
    *out = a;
    return MR_OK;
}

mr_status mr_adopted_affine_weight(const mr_adopted_affine* a, mr_affine_weight* out) {
    std::lock_guard<std::mutex> lock(g_mu);
    if (!a || !out || !registry().count(a))
        return fail(MR_INVALID_ARGUMENT, "mr_adopted_affine_weight: not a live adopted weight");
    *out = a->w;
    return MR_OK;
}

mr_status mr_adopted_affine_retain(mr_adopted_affine* a) {
    std::lock_guard<std::mutex> lock(g_mu);
    if (!a || !registry().count(a)) return fail(MR_INVALID_ARGUMENT, "mr_adopted_affine_retain: not a live adopted weight");
    ++a->refs;
    return MR_OK;
}

mr_status mr_adopted_affine_release(mr_adopted_affine* a, void* stream) {
    hipStream_t s = static_cast<hipStream_t>(stream);  // NULL: the default stream
    {
        // a host function recorded into a graph would run on every replay
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        const hipError_t e = hipStreamIsCapturing(s, &cap);
        if (e != hipSuccess) return hip_fail(e, "adopted weight release");
        if (cap != hipStreamCaptureStatusNone)
            return fail(MR_INVALID_ARGUMENT,
                        "mr_adopted_affine_release: the stream is capturing a graph; release on a stream that runs "
                        "the work directly");
    }
    bool last = false;
    mr_status st = drop_ref(a, "mr_adopted_affine_release", &last);
    if (st != MR_OK || !last) return st;
    if (hipLaunchHostFunc(s, finish, a) == hipSuccess) return MR_OK;
    (void)hipGetLastError();
    // the stream takes no host function: wait for its reads, then release here
    const hipError_t e = hipStreamSynchronize(s);
    finish(a);
    return e == hipSuccess ? MR_OK : hip_fail(e, "adopted weight release");
}

mr_status mr_adopted_affine_release_now(mr_adopted_affine* a) {
    bool last = false;
    mr_status st = drop_ref(a, "mr_adopted_affine_release_now", &last);
    if (st == MR_OK && last) finish(a);
    return st;
}

}  // extern "C"
