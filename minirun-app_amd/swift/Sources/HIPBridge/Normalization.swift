// K3Norm (ModelAdapters/Operators/Normalization.swift) over mr_rmsnorm.
import CMinirunHIP

/// K3Norm.rms(_:weight:eps:) (Normalization.swift:15-19):
/// weight * (x * rsqrt(mean(x^2) + eps)) over the last axis, fp32 arithmetic.
public func hipRMSNorm(_ x: HIPTensor, weight: HIPTensor, eps: Float, into out: HIPTensor,
                       stream: HIPStream = nil) throws {
    let dim = x.shape[x.shape.count - 1]
    let rows = x.shape.dropLast().reduce(1, *)
    try HIPError.check(mr_rmsnorm(x.raw, x.dtype, Int64(rows), Int32(dim), Int64(x.strides[x.strides.count - 2]),
                                  weight.raw, weight.dtype, eps, out.pointer, out.dtype,
                                  Int64(out.strides[out.strides.count - 2]), stream))
}
