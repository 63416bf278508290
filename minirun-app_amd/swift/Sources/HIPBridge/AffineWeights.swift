// MLX affine quantized weights on the device: the MLXBridge surface
// (Sources/MLXBridge/AffineWeights.swift) over mr_affine_*.
import CMinirunHIP

/// AffineWeights.init(packed:scales:biases:groupSize:bits:)
/// (MLXBridge/AffineWeights.swift:84-157): the same checks, in the same
/// order, with the same messages (mr_affine_validate).
public struct HIPAffineWeights {
    public let desc: mr_affine_weight
    public let experts: Int?

    public init(packed: HIPTensor, scales: HIPTensor, biases: HIPTensor, groupSize: Int, bits: Int) throws {
        var ex: Int64 = 0, outF: Int64 = 0, inF: Int64 = 0
        let ps = packed.shape.map(Int64.init), ss = scales.shape.map(Int64.init), bs = biases.shape.map(Int64.init)
        try HIPError.check(mr_affine_validate(packed.dtype, Int32(ps.count), ps, scales.dtype, Int32(ss.count), ss,
                                              biases.dtype, Int32(bs.count), bs, Int32(groupSize), Int32(bits),
                                              &ex, &outF, &inF))
        desc = mr_affine_weight(packed: packed.pointer.assumingMemoryBound(to: UInt32.self),
                                scales: UnsafeRawPointer(scales.pointer), biases: UnsafeRawPointer(biases.pointer),
                                scale_dtype: scales.dtype, out_features: outF, in_features: inF,
                                group: Int32(groupSize), bits: Int32(bits))
        experts = ex > 0 ? Int(ex) : nil
    }

    init(desc: mr_affine_weight) {
        self.desc = desc
        experts = nil
    }
}

/// affineMM(_:_:stream:) (MLXBridge/AffineWeights.swift:239-254):
/// y = x . dequant(W)^T, transpose fixed.
public func hipAffineMM(_ x: HIPTensor, _ w: HIPAffineWeights, into y: HIPTensor, stream: HIPStream = nil) throws {
    var d = w.desc
    try HIPError.check(mr_affine_matmul(x.raw, x.dtype, Int32(x.shape[0]), Int64(x.strides[0]), &d,
                                        y.pointer, y.dtype, Int64(y.strides[0]), stream))
}

/// affineGatherMM(_:_:rhsIndices:sortedIndices:stream:)
/// (MLXBridge/AffineWeights.swift:255-318): y[t, j] = W[rhs[t, j]] . x[t];
/// `w` is one expert of a stack of `experts`.
public func hipAffineGatherMM(_ x: HIPTensor, _ w: HIPAffineWeights, experts: Int, rhsIndices: HIPTensor,
                              into y: HIPTensor, stream: HIPStream = nil) throws {
    var d = w.desc
    try HIPError.check(mr_affine_gather_matmul(x.raw, x.dtype, Int32(x.shape[0]), Int64(x.strides[0]), &d,
                                               Int64(experts),
                                               UnsafePointer(rhsIndices.pointer.assumingMemoryBound(to: Int32.self)),
                                               Int32(rhsIndices.shape[1]), y.pointer, y.dtype, stream))
}

/// affineDequantize(_:dtype:stream:) (MLXBridge/AffineWeights.swift:328-342):
/// dense [out, in], f32 bit-exact or its bf16 rounding.
public func hipAffineDequantize(_ w: HIPAffineWeights, into out: HIPTensor, stream: HIPStream = nil) throws {
    var d = w.desc
    try HIPError.check(mr_affine_dequantize(&d, out.pointer, out.dtype, stream))
}

/// A StorageCore affine tile slot [packed | scales | biases]
/// (StorageCore/QuantizedTileContainer.swift:219-343) used in place as a
/// weight, as AffineWeights.adopting (:159-198) adopts the slot's bytes.
public struct HIPAffineTile {
    public let weights: HIPAffineWeights
    public let tileBytes: Int

    public init(slot: UnsafeRawPointer, rows: Int, cols: Int, groupSize: Int = 64, bits: Int = 4,
                scaleDType: mr_dtype = MR_BF16) throws {
        var d = mr_affine_weight()
        var n: Int64 = 0
        try HIPError.check(mr_affine_tile_view(slot, Int64(rows), Int64(cols), Int32(groupSize), Int32(bits),
                                               scaleDType, &d, &n))
        weights = HIPAffineWeights(desc: d)
        tileBytes = Int(n)
    }

    /// The slot from a pinned BufferPool lease to HBM, asynchronously on
    /// `stream` (release the lease once the stream has passed the copy).
    public static func upload(_ pinned: UnsafeRawPointer, to device: UnsafeMutableRawPointer, bytes: Int,
                              stream: HIPStream = nil) throws {
        try HIPError.check(mr_tile_upload(device, pinned, Int64(bytes), stream))
    }
}

/// A finalizer handed to the library: the Swift closure boxed as the C
/// callback's context, freed once the callback has run it.
private final class HIPFinalizerBox {
    let run: () -> Void
    init(_ run: @escaping () -> Void) { self.run = run }
}

private let hipRunFinalizer: mr_finalizer = { context in
    guard let context else { return }
    let box = Unmanaged<HIPFinalizerBox>.fromOpaque(context).takeRetainedValue()
    box.run()
}

/// AffineWeights.adopting(packedPointer:scalesPointer:biasesPointer:scaleDType:experts:outFeatures:
/// inFeatures:groupSize:bits:packedFinalizer:scalesFinalizer:biasesFinalizer:)
/// (MLXBridge/AffineWeights.swift:159-198): ownership of the three buffers
/// passes to the weight.  Each finalizer runs exactly once, after the last
/// reference is released and the named stream has passed every read, on a
/// HIP runtime thread or the releasing one (BufferPool.swift:45-90 releases
/// leases from such callbacks); a failed adoption runs them before throwing,
/// as the reference's arrays own the pointers before its validation.
public final class HIPAdoptedAffineWeights {
    public let handle: OpaquePointer
    public let weights: HIPAffineWeights

    public init(packedPointer: UnsafeMutableRawPointer, scalesPointer: UnsafeMutableRawPointer,
                biasesPointer: UnsafeMutableRawPointer, scaleDType: mr_dtype, experts: Int? = nil,
                outFeatures: Int, inFeatures: Int, groupSize: Int, bits: Int,
                packedFinalizer: @escaping () -> Void, scalesFinalizer: @escaping () -> Void,
                biasesFinalizer: @escaping () -> Void) throws {
        let ctx = [packedFinalizer, scalesFinalizer, biasesFinalizer].map {
            Unmanaged.passRetained(HIPFinalizerBox($0)).toOpaque()
        }
        var h: OpaquePointer?
        try HIPError.check(mr_affine_adopt(packedPointer, scalesPointer, biasesPointer, scaleDType,
                                           Int64(experts ?? 0), Int64(outFeatures), Int64(inFeatures),
                                           Int32(groupSize), Int32(bits), hipRunFinalizer, ctx[0],
                                           hipRunFinalizer, ctx[1], hipRunFinalizer, ctx[2], &h))
        handle = h!
        var d = mr_affine_weight()
        try HIPError.check(mr_adopted_affine_weight(handle, &d))
        weights = HIPAffineWeights(desc: d)
    }

    /// Another holder of the weight (a copy of the AffineWeights value in
    /// the reference, AffineWeights.swift:171-198).
    public func retain() throws {
        try HIPError.check(mr_adopted_affine_retain(handle))
    }

    /// Drops one holder; the last one runs the finalizers behind the work
    /// already enqueued on `stream` (nil is the default stream, as in every
    /// other call; the stream must carry every read of the weight).
    public func release(after stream: HIPStream) throws {
        try HIPError.check(mr_adopted_affine_release(handle, stream))
    }

    /// Drops one holder; the last one runs the finalizers before this
    /// returns.  For a weight no GPU work reads any more.
    public func releaseNow() throws {
        try HIPError.check(mr_adopted_affine_release_now(handle))
    }
}
