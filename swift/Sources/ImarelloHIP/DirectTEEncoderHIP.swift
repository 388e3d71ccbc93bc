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
/// (`embedRow`, :106-123, on the device by imq_dequantize), and
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
    let embed: ProjectionQ
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
        embed = try ProjectionQ(ctx, st, "embed_tokens", dtype: IMQ_BF16)
        var h: OpaquePointer?
        try ctx.check(imq_te_create(ctx.ctx, &weights, Int32(weights.count), Int32(Self.maxLen), 1e-6, &h))
        plan = h!
        x = try DeviceBuffer(ctx, bytes: Self.maxLen * Self.hidden * 2)
        y = try DeviceBuffer(ctx, bytes: Self.maxLen * Self.hidden * 2)
        qkv = try DeviceBuffer(ctx, bytes: Self.maxLen * Self.qkvWidth * 2)
        attnO = try DeviceBuffer(ctx, bytes: Self.maxLen * Self.nq * 2)
    }

    deinit { imq_te_destroy(plan) }

    /// `embedRow` for each token: the dequantized embedding row (bf16,
    /// RNE(s q + b), bit-exact with the reference's CPU form) into row `pos`.
    func embed(tokens: [Int32]) throws {
        let q = embed.q
        let k = Int(q.k)
        for (pos, t) in tokens.enumerated() {
            let row = Int(t)
            let w = q.w + row * (k / 8)
            let s = q.scales + row * (k / 64) * 2
            let b = q.biases + row * (k / 64) * 2
            try ctx.check(imq_dequantize(ctx.ctx, w, s, b, x.at(pos * k * 2), q.k, 1, 64, 4, IMQ_BF16,
                                         ctx.stream))
        }
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
