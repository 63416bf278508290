// K3MLA (ModelAdapters/Operators/MLA.swift): the latent cache, the absorbed
// decode attention, the whole decode block, the eager prefill and the whole
// prefill block.
import CMinirunHIP

/// The latent cache of K3MLA.State (MLA.swift:28-36): normalized latents
/// [positions, 512] and the shared rope keys [positions, 64], bf16; both may
/// be views of one [positions, 576] buffer.
public struct HIPLatentCache {
    public var latents: HIPTensor
    public var sharedKeys: HIPTensor
    public var count: Int  // positions written
}

/// The append of K3MLA.forward (MLA.swift:142-157): RMSNorm of the kv_a
/// row's latent part and its rope slice (rotated with cos/sin, or stored
/// as it is when both are nil: K3 is NoPE, MLA.swift:5-13) into the cache.
public func hipMLACacheAppend(_ kv: HIPTensor, normWeight: HIPTensor, eps: Float, cos: UnsafePointer<Float>?,
                              sin: UnsafePointer<Float>?, cache: inout HIPLatentCache, stream: HIPStream = nil) throws {
    let tokens = kv.shape[0]
    try HIPError.check(mr_mla_cache_append(kv.raw, kv.dtype, Int64(kv.strides[0]), Int64(tokens), normWeight.raw,
                                           normWeight.dtype, eps, 512, 64, cos, sin, cache.latents.pointer,
                                           Int64(cache.latents.strides[0]), cache.sharedKeys.pointer,
                                           Int64(cache.sharedKeys.strides[0]), Int64(cache.count), stream))
    cache.count += tokens
}

/// latentQueries = qPass . keyProjection (MLA.swift:180-188); kv_b dense
/// (K3) or affine.
public func hipMLAAbsorbQuery(_ q: HIPTensor, heads: Int, nopeDim: Int, vDim: Int, kvB: HIPProjection,
                              into qLat: HIPTensor, stream: HIPStream = nil) throws {
    var p = kvB.desc
    try HIPError.check(mr_mla_absorb_query(q.raw, Int64(q.strides[0]), Int32(heads), Int32(nopeDim), Int32(vDim),
                                           &p, qLat.pointer, Int64(qLat.strides[0]), stream))
}

/// attention = latentOutput . valueProjection^T (MLA.swift:196-197).
public func hipMLAUnabsorbValues(_ ctx: HIPTensor, heads: Int, nopeDim: Int, vDim: Int, kvB: HIPProjection,
                                 into out: HIPTensor, stream: HIPStream = nil) throws {
    var p = kvB.desc
    try HIPError.check(mr_mla_unabsorb_values(ctx.raw, Int64(ctx.strides[0]), Int32(heads), Int32(nopeDim),
                                              Int32(vDim), &p, out.pointer, out.dtype, stream))
}

/// The absorbed attention core of K3MLA.forwardWithoutTrace
/// (MLA.swift:188-197): softmax((q_lat . c + q_rope . k_rot) * scale) . c
/// over the cache rows, per (batch, head); out [batch, heads, 512].
/// `workspace` comes from hipMLADecodeWorkspaceSize; nil runs the
/// library's no-allocation entry point (for graph capture).
public func hipMLADecode(qLat: HIPTensor, qRope: HIPTensor, cache: HIPLatentCache, scale: Float, into out: HIPTensor,
                         workspace: HIPTensor?, stream: HIPStream = nil) throws {
    var a = decodeArgs(qLat: qLat, qRope: qRope, cache: cache, scale: scale, out: out)
    guard let ws = workspace else {
        try HIPError.check(mr_mla_decode_noalloc(&a, stream))
        return
    }
    a.workspace = ws.pointer
    a.workspace_bytes = ws.shape[0]
    try HIPError.check(mr_mla_decode(&a, stream))
}

/// Bytes of device scratch hipMLADecode needs for these shapes
/// (mr_mla_decode_workspace_size; reusable across calls on one stream).
public func hipMLADecodeWorkspaceSize(qLat: HIPTensor, qRope: HIPTensor, cache: HIPLatentCache, scale: Float,
                                      out: HIPTensor) -> Int {
    var a = decodeArgs(qLat: qLat, qRope: qRope, cache: cache, scale: scale, out: out)
    return mr_mla_decode_workspace_size(&a)
}

func decodeArgs(qLat: HIPTensor, qRope: HIPTensor, cache: HIPLatentCache, scale: Float,
                out: HIPTensor) -> mr_mla_decode_args {
    var a = mr_mla_decode_args()
    a.batch = Int32(qLat.shape[0]); a.heads = Int32(qLat.shape[1]); a.n_ctx = Int32(cache.count)
    a.kv_rank = 512; a.rope_dim = 64; a.scale = scale
    a.q_lat = qLat.raw; a.q_lat_batch_stride = Int64(qLat.strides[0]); a.q_lat_head_stride = Int64(qLat.strides[1])
    a.q_rope = qRope.raw; a.q_rope_batch_stride = Int64(qRope.strides[0])
    a.q_rope_head_stride = Int64(qRope.strides[1])
    a.latent = cache.latents.raw; a.latent_row_stride = Int64(cache.latents.strides[0])
    a.rope_keys = cache.sharedKeys.raw; a.rope_row_stride = Int64(cache.sharedKeys.strides[0])
    a.out = out.pointer; a.out_dtype = out.dtype
    a.out_batch_stride = Int64(out.strides[0]); a.out_head_stride = Int64(out.strides[1])
    return a
}

/// K3MLA.Weights (MLA.swift:38-47) for the block, with optional RMSNorm
/// weights (input_layernorm is applied by K3 before the block: nil here).
public struct HIPMLABlockWeights {
    public var inputNorm: HIPTensor?
    public var qALayerNorm: HIPTensor
    public var kvALayerNorm: HIPTensor
    public var qAProj, qBProj, kvAProjWithMQA, kvBProj, oProj: HIPProjection
    public var gProj: HIPProjection?  // the output gate (mla_use_output_gate)
}

/// One decode token through K3MLA.forwardWithoutTrace (MLA.swift:91-98 ->
/// :124-229): projections, cache append at `position`, absorbed attention,
/// gate and o_proj.  cos/sin nil = NoPE (K3).
public func hipMLADecodeBlock(_ x: HIPTensor, weights w: HIPMLABlockWeights, hidden: Int, qLoraRank: Int,
                              heads: Int, eps: Float, cache: inout HIPLatentCache, capacity: Int,
                              cos: UnsafePointer<Float>?, sin: UnsafePointer<Float>?, into out: HIPTensor,
                              workspace: HIPTensor, stream: HIPStream = nil) throws {
    var a = mr_mla_block_args()
    a.hidden = Int32(hidden); a.q_lora_rank = Int32(qLoraRank); a.heads = Int32(heads)
    a.qk_nope_dim = 128; a.qk_rope_dim = 64; a.v_head_dim = 128; a.kv_rank = 512
    a.eps = eps; a.scale = Float(1.0 / (192.0).squareRoot())  // over the full query (MLA.swift:170)
    a.x = x.raw
    a.input_norm_w = w.inputNorm.map { $0.raw }
    a.q_a_norm_w = w.qALayerNorm.raw; a.kv_a_norm_w = w.kvALayerNorm.raw
    a.norm_w_dtype = w.qALayerNorm.dtype
    a.q_a = w.qAProj.desc; a.q_b = w.qBProj.desc; a.kv_a = w.kvAProjWithMQA.desc
    a.kv_b = w.kvBProj.desc; a.o_proj = w.oProj.desc
    a.g_proj = w.gProj?.desc ?? HIPProjection.absent()
    a.cache_latent = cache.latents.pointer; a.latent_row_stride = Int64(cache.latents.strides[0])
    a.cache_rope = cache.sharedKeys.pointer; a.rope_row_stride = Int64(cache.sharedKeys.strides[0])
    a.position = Int32(cache.count); a.capacity = Int32(capacity)
    a.rope_cos = cos; a.rope_sin = sin
    a.out = out.pointer
    a.workspace = workspace.pointer; a.workspace_bytes = workspace.shape[0]
    guard a.workspace_bytes >= mr_mla_decode_block_workspace_size(&a) else {
        throw HIPError(status: MR_WORKSPACE_TOO_SMALL, description: "decode block workspace too small")
    }
    try HIPError.check(mr_mla_decode_block(&a, stream))
    cache.count += 1
}

/// K3MLA.forward's eager prefill (MLA.swift:159-168,198-206; expand
/// :231-245; causal mask :257-275): q [T, H, 192], kv_b dense [H*256, 512].
public func hipMLAPrefill(q: HIPTensor, cache: HIPLatentCache, kvB: HIPTensor, scale: Float, into out: HIPTensor,
                          workspace: HIPTensor, stream: HIPStream = nil) throws {
    var a = mr_mla_prefill_args()
    a.tokens = Int32(q.shape[0]); a.n_ctx = Int32(cache.count); a.heads = Int32(q.shape[1])
    a.qk_nope_dim = 128; a.qk_rope_dim = 64; a.v_head_dim = 128; a.kv_rank = 512; a.scale = scale
    a.q = q.raw; a.q_token_stride = Int64(q.strides[0]); a.q_head_stride = Int64(q.strides[1])
    a.latent = cache.latents.raw; a.latent_row_stride = Int64(cache.latents.strides[0])
    a.rope_keys = cache.sharedKeys.raw; a.rope_row_stride = Int64(cache.sharedKeys.strides[0])
    a.kv_b = kvB.raw; a.kv_b_row_stride = Int64(kvB.strides[0])
    a.out = out.pointer; a.out_dtype = out.dtype
    a.out_token_stride = Int64(out.strides[0]); a.out_head_stride = Int64(out.strides[1])
    a.workspace = workspace.pointer; a.workspace_bytes = workspace.shape[0]
    guard a.workspace_bytes >= mr_mla_prefill_workspace_size(&a) else {
        throw HIPError(status: MR_WORKSPACE_TOO_SMALL, description: "prefill workspace too small")
    }
    try HIPError.check(mr_mla_prefill(&a, stream))
}

/// K3MLA.forward over a whole prompt in one call (MLA.swift:124-229): the T
/// rows of x [T, hidden] through the projections, the cache append at rows
/// cache.count ..< cache.count + T (state == nil is an empty cache), the
/// eager causal attention, the gate and o_proj; out [T, hidden] bf16.
/// cos/sin: device [T, 32] tables at those positions, nil = NoPE (K3).
/// `workspace` comes from hipMLAPrefillBlockWorkspaceSize.
public func hipMLAPrefillBlock(_ x: HIPTensor, weights w: HIPMLABlockWeights, qLoraRank: Int, heads: Int, eps: Float,
                               cache: inout HIPLatentCache, capacity: Int, cos: UnsafePointer<Float>?,
                               sin: UnsafePointer<Float>?, into out: HIPTensor, workspace: HIPTensor,
                               stream: HIPStream = nil) throws {
    var a = prefillBlockArgs(x, weights: w, qLoraRank: qLoraRank, heads: heads, eps: eps, cache: cache,
                             capacity: capacity, cos: cos, sin: sin, out: out)
    a.workspace = workspace.pointer; a.workspace_bytes = workspace.shape[0]
    guard a.workspace_bytes >= mr_mla_prefill_block_workspace_size(&a) else {
        throw HIPError(status: MR_WORKSPACE_TOO_SMALL, description: "prefill block workspace too small")
    }
    try HIPError.check(mr_mla_prefill_block(&a, stream))
    cache.count += x.shape[0]
}

/// Bytes of device scratch hipMLAPrefillBlock needs for this prompt.
public func hipMLAPrefillBlockWorkspaceSize(_ x: HIPTensor, weights w: HIPMLABlockWeights, qLoraRank: Int, heads: Int,
                                            cache: HIPLatentCache, out: HIPTensor) -> Int {
    var a = prefillBlockArgs(x, weights: w, qLoraRank: qLoraRank, heads: heads, eps: 0, cache: cache,
                             capacity: cache.count + x.shape[0], cos: nil, sin: nil, out: out)
    return mr_mla_prefill_block_workspace_size(&a)
}

func prefillBlockArgs(_ x: HIPTensor, weights w: HIPMLABlockWeights, qLoraRank: Int, heads: Int, eps: Float,
                      cache: HIPLatentCache, capacity: Int, cos: UnsafePointer<Float>?, sin: UnsafePointer<Float>?,
                      out: HIPTensor) -> mr_mla_prefill_block_args {
    var a = mr_mla_prefill_block_args()
    a.tokens = Int32(x.shape[0]); a.hidden = Int32(x.shape[1])
    a.q_lora_rank = Int32(qLoraRank); a.heads = Int32(heads)
    a.qk_nope_dim = 128; a.qk_rope_dim = 64; a.v_head_dim = 128; a.kv_rank = 512
    a.eps = eps; a.scale = Float(1.0 / (192.0).squareRoot())  // over the full query (MLA.swift:170)
    a.x = x.raw; a.x_token_stride = Int64(x.strides[0])
    a.input_norm_w = w.inputNorm.map { $0.raw }
    a.q_a_norm_w = w.qALayerNorm.raw; a.kv_a_norm_w = w.kvALayerNorm.raw
    a.norm_w_dtype = w.qALayerNorm.dtype
    a.q_a = w.qAProj.desc; a.q_b = w.qBProj.desc; a.kv_a = w.kvAProjWithMQA.desc
    a.kv_b = w.kvBProj.desc; a.o_proj = w.oProj.desc
    a.g_proj = w.gProj?.desc ?? HIPProjection.absent()
    a.cache_latent = cache.latents.pointer; a.latent_row_stride = Int64(cache.latents.strides[0])
    a.cache_rope = cache.sharedKeys.pointer; a.rope_row_stride = Int64(cache.sharedKeys.strides[0])
    a.position = Int32(cache.count); a.capacity = Int32(capacity)
    a.rope_cos = cos; a.rope_sin = sin
    a.out = out.pointer; a.out_token_stride = Int64(out.strides[0])
    return a
}
