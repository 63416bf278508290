// DeepSeekV4LightningIndexer (ModelAdapters/Operators/DeepSeekV4Attention.swift:526-645).
import CMinirunHIP

/// DeepSeekV4LightningIndexer.scores(queries:compressedKeys:headWeights:)
/// (DeepSeekV4Attention.swift:530-549): [S, T] f32 scores on the device.
public func hipLightningScores(queries q: HIPTensor, compressedKeys k: HIPTensor, headWeights w: HIPTensor,
                               into out: HIPTensor, stream: HIPStream = nil) throws {
    try HIPError.check(mr_indexer_scores(q.raw, q.dtype, Int32(q.shape[0]), Int32(q.shape[1]), Int32(q.shape[2]),
                                         Int64(q.strides[0]), Int64(q.strides[1]), k.raw, k.dtype, Int32(k.shape[0]),
                                         Int32(k.shape[1]), Int64(k.strides[0]), w.raw, w.dtype, Int32(w.shape[0]),
                                         Int32(w.shape[1]), Int64(w.strides[0]),
                                         out.pointer.assumingMemoryBound(to: Float.self), Int64(out.strides[0]),
                                         stream))
}

/// DeepSeekV4LightningIndexer.select(scores:topK:ratio:startPosition:offset:)
/// (DeepSeekV4Attention.swift:554-645): [rows, selected] int32 key indices
/// on the device (offset + key, -1 past the visible keys), bit-exact with
/// the reference's order.  With `status` the NaN report stays on the device;
/// without it the call throws the reference's NaN error (one sync).
/// Returns the number of keys each row received.
@discardableResult
public func hipLightningSelect(scores: HIPTensor, topK: Int, ratio: Int, startPosition: Int, offset: Int,
                               into out: HIPTensor, status: UnsafeMutablePointer<Int32>?, workspace: HIPTensor,
                               stream: HIPStream = nil) throws -> Int {
    let rows = Int32(scores.shape[0]), cols = Int32(scores.shape[1])
    var selected: Int32 = 0
    try HIPError.check(mr_topk_geometry(rows, cols, Int32(topK), Int32(ratio), Int32(startPosition), Int32(offset),
                                        &selected))
    guard workspace.shape[0] >= mr_topk_workspace_size(rows, cols, Int32(topK)) else {
        throw HIPError(status: MR_WORKSPACE_TOO_SMALL, description: "selection workspace too small")
    }
    var a = mr_topk_args(scores: UnsafePointer(scores.pointer.assumingMemoryBound(to: Float.self)),
                         score_row_stride: Int64(scores.strides[0]), rows: rows, cols: cols, top_k: Int32(topK),
                         ratio: Int32(ratio), start_pos: Int32(startPosition), offset: Int32(offset),
                         out: out.pointer.assumingMemoryBound(to: Int32.self), out_row_stride: Int64(out.strides[0]),
                         status: status, flags: 0, workspace: workspace.pointer, workspace_bytes: workspace.shape[0])
    try HIPError.check(mr_topk_select(&a, stream))
    return Int(selected)
}
