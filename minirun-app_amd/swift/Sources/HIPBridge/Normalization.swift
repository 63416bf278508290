// K3Norm (ModelAdapters/Operators/Normalization.swift) over mr_rmsnorm.
import CMinirunHIP

/// K3Norm.rms(_:weight:eps:) (Normalization.swift:15-19):
/// weight * (x * rsqrt(mean(x^2) + eps)) over the last axis, fp32 arithmetic.
public func hipRMSNorm(_ x: HIPTensor, weight: HIPTensor, eps: Float, into out: HIPTensor,
                       stream: HIPStream = nil) throws {
    let dim = x.shape[x.shape.count - 1]
    let rows = x.shape.dropLast().reduce(1, *)
    // a 1-D tensor is one row: its row stride is never used, take the width
    let xRowStride = x.strides.count > 1 ? x.strides[x.strides.count - 2] : dim
    let outRowStride = out.strides.count > 1 ? out.strides[out.strides.count - 2] : dim
    try HIPError.check(mr_rmsnorm(x.raw, x.dtype, Int64(rows), Int32(dim), Int64(xRowStride),
                                  weight.raw, weight.dtype, eps, out.pointer, out.dtype,
                                  Int64(outRowStride), stream))
}
