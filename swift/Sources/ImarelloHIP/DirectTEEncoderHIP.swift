import CImq

/// The attention core of a text-encoder layer (per-head q / k norms, RoPE and
/// masked or causal attention, DirectTEEncoder.swift:382-389): not quantized-
/// linear work, so the caller provides it.  It reads q | k | v (columns
/// [0, 4096), [4096, 5120), [5120, 6144) of `qkv`, T [rows, 6144]) and writes
/// `attnO` (T [rows, 4096]), on the context's stream.
public protocol TEAttentionCore: AnyObject {
    func attend(layer: Int, qkv: DeviceBuffer, rows: Int, attnO: DeviceBuffer) throws
}

/// `DirectTEEncoder` (Sources/ImarelloDirect/DirectTEEncoder.swift) over include/imq_te.h:
/// the layers `DirectTEForward.loadLayers` uploads (DirectTEForward.swift:97-138, raw
/// bf16 parameters, q/k/v and gate/up concatenated), the embedding rows
/// (`embedRow`, :106-123, on the device by imq_dequantize_rows), and
/// `encode` / `encodeRealOnly` (:249-360) as the 27-layer loop with the
/// hidden-state taps after layers 9, 18 and 27 (DirectTEForward.swift:20).
public final class DirectTEEncoderHIP {
    public static let hidden = 2560
    public static let nLayers = 27
    public static let taps = [9, 18, 27]
    public static let maxLen = 512
    static let qkvWidth = 6144
    static let nq = 4096

    public let ctx: HIPContext
    var layers: [[ProjectionQ]] = []  // qkv, o, gate_up, down
    var norms: [(DeviceBuffer, DeviceBuffer)] = []
    let embedTable: ProjectionQ
    let plan: OpaquePointer
    let x, y, qkv, attnO: DeviceBuffer

    public init(textEncoderDirectory: String, context: HIPContext? = nil) throws {
        ctx = try context ?? HIPContext()
        let st = try SafetensorsHIP(directory: textEncoderDirectory)
        var weights: [imq_te_layer_weights] = []
        for i in 0 ..< Self.nLayers {
            let p = "layers.\(i)"
            let qkvQ = try ProjectionQ(ctx, st, prefixes: ["\(p).self_attn.q_proj", "\(p).self_attn.k_proj",
                                                           "\(p).self_attn.v_proj"], dtype: IMQ_BF16)
            let o = try ProjectionQ(ctx, st, "\(p).self_attn.o_proj", dtype: IMQ_BF16)
            let gu = try ProjectionQ(ctx, st, prefixes: ["\(p).mlp.gate_proj", "\(p).mlp.up_proj"],
                                     dtype: IMQ_BF16)
            let down = try ProjectionQ(ctx, st, "\(p).mlp.down_proj", dtype: IMQ_BF16)
            let nIn = try st.uploadF32(ctx, "\(p).input_layernorm.weight", count: Self.hidden)
            let nPost = try st.uploadF32(ctx, "\(p).post_attention_layernorm.weight", count: Self.hidden)
            layers.append([qkvQ, o, gu, down])
            norms.append((nIn, nPost))
            weights.append(imq_te_layer_weights(
                qkv: qkvQ.q, o: o.q, gate_up: gu.q, down: down.q,
                norm_in: nIn.ptr.assumingMemoryBound(to: Float.self),
                norm_post: nPost.ptr.assumingMemoryBound(to: Float.self)))
        }
        embedTable = try ProjectionQ(ctx, st, "embed_tokens", dtype: IMQ_BF16)
        var h: OpaquePointer?
        try ctx.check(imq_te_create(ctx.ctx, &weights, Int32(weights.count), Int32(Self.maxLen), 1e-6, &h))
        plan = h!
        x = try DeviceBuffer(ctx, bytes: Self.maxLen * Self.hidden * 2)
        y = try DeviceBuffer(ctx, bytes: Self.maxLen * Self.hidden * 2)
        qkv = try DeviceBuffer(ctx, bytes: Self.maxLen * Self.qkvWidth * 2)
        attnO = try DeviceBuffer(ctx, bytes: Self.maxLen * Self.nq * 2)
    }

    deinit { imq_te_destroy(plan) }

    /// `embedRow` for every token in one launch: the dequantized embedding rows
    /// (bf16, RNE(s q + b), bit-exact with the reference's CPU form) into x.
    func embed(tokens: [Int32]) throws {
        let q = embedTable.q
        guard tokens.allSatisfy({ $0 >= 0 && $0 < q.n }) else {
            throw HIPError.shape("token id outside [0, \(q.n))")
        }
        let ids = try DeviceBuffer(ctx, copying: tokens)
        try ctx.check(imq_dequantize_rows(ctx.ctx, q.w, q.scales, q.biases,
                                          ids.ptr.assumingMemoryBound(to: Int32.self),
                                          Int32(tokens.count), x.ptr, q.k, q.n, 64, 4, IMQ_BF16,
                                          ctx.stream))
        try ctx.sync()  // ids is released on return
    }

    /// The layer loop of `encode` / `encodeRealOnly` over `tokens` (the
    /// chat-templated ids; the tokenizer stays the caller's): per layer
    /// `imq_te_attn_in`, the caller's attention core, `imq_te_attn_out_mlp`;
    /// returns the three tapped hidden states, bf16 [rows, 2560] each.
    public func encode(tokens: [Int32], attention: TEAttentionCore) throws -> [[UInt16]] {
        let rows = tokens.count
        guard rows > 0 && rows <= Self.maxLen else { throw HIPError.shape("\(rows) tokens") }
        try embed(tokens: tokens)
        var cur = x, alt = y
        var out: [[UInt16]] = []
        for li in 0 ..< Self.nLayers {
            try ctx.check(imq_te_attn_in(plan, Int32(li), cur.ptr, qkv.ptr, Int32(rows), ctx.stream))
            try attention.attend(layer: li, qkv: qkv, rows: rows, attnO: attnO)
            try ctx.check(imq_te_attn_out_mlp(plan, Int32(li), cur.ptr, attnO.ptr, alt.ptr, Int32(rows),
                                              ctx.stream))
            swap(&cur, &alt)
            if Self.taps.contains(li + 1) {
                out.append(try cur.download(UInt16.self, count: rows * Self.hidden))
            }
        }
        return out
    }
}
