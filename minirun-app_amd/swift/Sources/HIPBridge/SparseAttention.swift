// DeepSeekV4SparseAttention and DeepSeekV4AttentionIndices
// (ModelAdapters/Operators/DeepSeekV4Attention.swift:169-237, 747-920).
import CMinirunHIP

/// DeepSeekV4SparseAttention.forward(queries:keysAndValues:sinks:indices:scale:)
/// (DeepSeekV4Attention.swift:747-770, batched form :861-920), MLA layout:
/// K = row[0:576], V = row[0:512] of per-sequence caches [B, N, 576]
/// (qRope nil and a [N, 512] cache: the V4 form, K = V = row).  The index
/// checks of :884-895 run on the device in the same launch and land in
/// `indexStatus` ([B][3] int32: status, position, value per token); with
/// indexStatus nil the call checks first and throws the reference's error.
public func hipSparseAttention(qLat: HIPTensor, qRope: HIPTensor?, cache: HIPTensor, indices: HIPTensor,
                               sinks: UnsafePointer<Float>?, scale: Float, into out: HIPTensor,
                               indexStatus: UnsafeMutablePointer<Int32>?, workspace: HIPTensor,
                               stream: HIPStream = nil) throws {
    var a = mr_mla_decode_args()
    let batched = cache.shape.count == 3
    a.batch = Int32(qLat.shape[0]); a.heads = Int32(qLat.shape[1])
    a.n_ctx = Int32(batched ? cache.shape[1] : cache.shape[0])
    a.kv_rank = 512; a.rope_dim = qRope == nil ? 0 : 64; a.scale = scale
    a.q_lat = qLat.raw; a.q_lat_batch_stride = Int64(qLat.strides[0]); a.q_lat_head_stride = Int64(qLat.strides[1])
    if let qRope {
        a.q_rope = qRope.raw; a.q_rope_batch_stride = Int64(qRope.strides[0])
        a.q_rope_head_stride = Int64(qRope.strides[1])
    }
    let rowStride = Int64(cache.strides[batched ? 1 : 0])
    let batchStride = batched ? Int64(cache.strides[0]) : 0
    a.latent = cache.raw; a.latent_row_stride = rowStride; a.latent_batch_stride = batchStride
    if qRope != nil {
        a.rope_keys = UnsafeRawPointer(cache.pointer.advanced(by: 512 * 2))
        a.rope_row_stride = rowStride; a.rope_batch_stride = batchStride
    }
    a.indices = UnsafePointer(indices.pointer.assumingMemoryBound(to: Int32.self))
    a.n_idx = Int32(indices.shape[1])
    a.sinks = sinks
    a.out = out.pointer; a.out_dtype = out.dtype
    a.out_batch_stride = Int64(out.strides[0]); a.out_head_stride = Int64(out.strides[1])
    a.index_status = indexStatus
    a.workspace = workspace.pointer; a.workspace_bytes = workspace.shape[0]
    guard a.workspace_bytes >= mr_mla_decode_workspace_size(&a) else {
        throw HIPError(status: MR_WORKSPACE_TOO_SMALL, description: "sparse attention workspace too small")
    }
    try HIPError.check(mr_mla_decode(&a, stream))
}

/// The index checks alone (DeepSeekV4Attention.swift:884-895), throwing the
/// reference's error for the first bad token; synchronises `stream`.
public func hipValidateIndices(_ indices: HIPTensor, rows: Int, workspace: HIPTensor,
                               stream: HIPStream = nil) throws {
    let b = Int32(indices.shape[0]), k = Int32(indices.shape[1])
    guard workspace.shape[0] >= mr_validate_indices_workspace_size(b, k) else {
        throw HIPError(status: MR_WORKSPACE_TOO_SMALL, description: "index validation workspace too small")
    }
    var token: Int32 = -1, position: Int32 = -1
    try HIPError.check(mr_validate_indices(UnsafePointer(indices.pointer.assumingMemoryBound(to: Int32.self)), b, k,
                                           Int32(rows), workspace.pointer, workspace.shape[0], &token, &position,
                                           stream))
}

/// DeepSeekV4AttentionIndices.window(size:sequenceLength:startPosition:)
/// (DeepSeekV4Attention.swift:170-198), on the host; -1 = invalid.
public func hipAttentionIndicesWindow(size: Int, sequenceLength: Int, startPosition: Int) throws -> [[Int32]] {
    let width = startPosition > 0 ? size : min(sequenceLength, size)
    var flat = [Int32](repeating: -1, count: max(sequenceLength * width, size))
    var rows: Int32 = 0, cols: Int32 = 0
    try HIPError.check(mr_attention_indices_window(Int32(size), Int32(sequenceLength), Int32(startPosition), &flat,
                                                   &rows, &cols))
    return (0..<Int(rows)).map { Array(flat[$0 * Int(cols)..<($0 + 1) * Int(cols)]) }
}

/// DeepSeekV4AttentionIndices.compressed(ratio:sequenceLength:startPosition:offset:)
/// (DeepSeekV4Attention.swift:200-228), on the host; -1 = invalid.
public func hipAttentionIndicesCompressed(ratio: Int, sequenceLength: Int, startPosition: Int,
                                          offset: Int) throws -> [[Int32]] {
    let width = max(sequenceLength / ratio, (startPosition + 1) / ratio, 1)
    var flat = [Int32](repeating: -1, count: max(sequenceLength, 1) * width)
    var rows: Int32 = 0, cols: Int32 = 0
    try HIPError.check(mr_attention_indices_compressed(Int32(ratio), Int32(sequenceLength), Int32(startPosition),
                                                       Int32(offset), &flat, &rows, &cols))
    return (0..<Int(rows)).map { Array(flat[$0 * Int(cols)..<($0 + 1) * Int(cols)]) }
}
