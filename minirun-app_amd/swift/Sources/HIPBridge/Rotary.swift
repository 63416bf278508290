// DeepSeekV4RotaryParameters / DeepSeekV4Rotary
// (ModelAdapters/Operators/DeepSeekV4Attention.swift:28-165).
import CMinirunHIP

/// DeepSeekV4RotaryParameters (DeepSeekV4Attention.swift:28-99): pair
/// frequencies base^(-2i/dim), with the YaRN ramp when originalLength > 0.
public struct HIPRotaryParameters {
    public let dimension: Int
    public let frequencies: [Double]

    public init(dimension: Int, base: Double = 10000, originalLength: Int = 0, factor: Double = 1,
                betaFast: Double = 32, betaSlow: Double = 1) throws {
        var f = [Double](repeating: 0, count: dimension / 2)
        try HIPError.check(mr_rope_frequencies(Int32(dimension), Int32(originalLength), base, factor, betaFast,
                                               betaSlow, &f))
        self.dimension = dimension
        frequencies = f
    }

    /// The fp32 cos/sin tables [positions, dimension/2] of fp64 angles
    /// (DeepSeekV4Attention.swift:126-149); `inverse` negates the angles.
    public func tables(positions: [Int], inverse: Bool = false) throws -> (cos: [Float], sin: [Float]) {
        let half = dimension / 2
        var c = [Float](repeating: 0, count: positions.count * half)
        var s = c
        let pos = positions.map(Int64.init)
        try HIPError.check(mr_rope_table(pos, Int64(pos.count), frequencies, Int32(half), inverse ? 1 : 0, &c, &s))
        return (c, s)
    }
}

/// DeepSeekV4Rotary.apply(_:positions:parameters:inverse:)
/// (DeepSeekV4Attention.swift:108-165), in place: x [positions, inner, row],
/// columns [col0, col0 + dim) as adjacent pairs, device tables cos/sin.
public func hipRotaryApply(_ x: HIPTensor, col0: Int, dimension: Int, cos: UnsafePointer<Float>,
                           sin: UnsafePointer<Float>, stream: HIPStream = nil) throws {
    let inner = x.shape.dropFirst().dropLast().reduce(1, *)
    try HIPError.check(mr_rope_apply(x.pointer, x.dtype, Int64(x.shape[0]), Int64(inner),
                                     Int64(x.shape[x.shape.count - 1]), Int64(col0), Int32(dimension), cos, sin,
                                     stream))
}
