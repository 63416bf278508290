// Dense projections (ModelAdapters/Operators/Linear.swift) over mr_linear,
// and the dense-or-quantized projection the MLA block takes.
import CMinirunHIP

/// A dense weight stored output-major [outFeatures, inFeatures], bf16 or f32.
public struct HIPDenseWeights {
    public let desc: mr_dense_weight

    public init(_ w: HIPTensor) {
        desc = mr_dense_weight(weight: w.raw, dtype: w.dtype, out_features: Int64(w.shape[0]),
                               in_features: Int64(w.shape[1]), row_stride: Int64(w.strides[0]))
    }
}

/// k3Linear(_:_:) (ModelAdapters/Operators/Linear.swift:55-57): y = x . W^T.
public func hipK3Linear(_ x: HIPTensor, _ w: HIPDenseWeights, into y: HIPTensor, stream: HIPStream = nil) throws {
    var d = w.desc
    try HIPError.check(mr_linear(x.raw, x.dtype, Int32(x.shape[0]), Int64(x.strides[0]), &d, y.pointer, y.dtype,
                                 Int64(y.strides[0]), stream))
}

/// K3Projection (ModelAdapters/Operators/Linear.swift:20-49): one storage
/// or the other; here the quantized form is MLX affine.
public enum HIPProjection {
    case dense(HIPDenseWeights)
    case affine(HIPAffineWeights)

    var desc: mr_projection {
        var p = mr_projection()
        switch self {
        case .dense(let w):
            p.kind = MR_PROJ_DENSE
            p.dense = w.desc
        case .affine(let w):
            p.kind = MR_PROJ_AFFINE
            p.affine = w.desc
        }
        return p
    }

    static func absent() -> mr_projection {
        var p = mr_projection()
        p.kind = MR_PROJ_NONE
        return p
    }
}
