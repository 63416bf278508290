// Device buffers and errors of the bridge.  An HIPTensor stands where MLX
// passes an MLXArray: caller-owned device memory (or pinned host memory the
// device reads), a shape and element strides, no ownership.
import CMinirunHIP

public typealias HIPStream = UnsafeMutableRawPointer?  // hipStream_t; nil = the default stream

public struct HIPTensor {
    public var pointer: UnsafeMutableRawPointer
    public var shape: [Int]
    public var strides: [Int]  // elements
    public var dtype: mr_dtype

    public init(pointer: UnsafeMutableRawPointer, shape: [Int], strides: [Int]? = nil, dtype: mr_dtype) {
        self.pointer = pointer
        self.shape = shape
        self.dtype = dtype
        if let strides {
            self.strides = strides
        } else {  // row-major
            var s = [Int](repeating: 1, count: shape.count)
            var acc = 1
            for i in stride(from: shape.count - 1, through: 0, by: -1) {
                s[i] = acc
                acc *= shape[i]
            }
            self.strides = s
        }
    }

    public var raw: UnsafeRawPointer { UnsafeRawPointer(pointer) }
    public func bytes(_ n: Int) -> Int { n * (dtype == MR_F32 || dtype == MR_U32 || dtype == MR_I32 ? 4 : 2) }
}

/// A non-OK mr_status with the library's message for it (the reference's
/// wording where it has one: AffineBridgeError, DeepSeekV4Error).
public struct HIPError: Error, CustomStringConvertible {
    public let status: mr_status
    public let description: String

    static func check(_ st: mr_status) throws {
        guard st != MR_OK else { return }
        throw HIPError(status: st, description: String(cString: mr_get_last_error()))
    }
}

/// Library identity, e.g. "minirun-hip 0.1.0 gfx950".
public var hipBridgeVersion: String { String(cString: mr_version()) }
