import CImq

/// One timestep's conditioning, the fields of `Flux2StepConditioning` that
/// `DirectConditioner.stepConditioning` fills (Sources/ImarelloDirect/DirectConditioner.swift:186-208),
/// as host floats: each triple is three consecutive dim-wide slices of a head.
public struct StepConditioningHIP {
    public var temb: [Float]
    public var doubleImg: [([Float], [Float], [Float])]
    public var doubleTxt: [([Float], [Float], [Float])]
    public var single: ([Float], [Float], [Float])
    public var outScale: [Float]
    public var outShift: [Float]
}

/// `DirectConditioner` (DirectConditioner.swift) over include/imq_cond.h and the bf16
/// qmm: `init(transformerDirectory:)` loads the same projections with f32
/// parameters (:75-95, the four modulation heads as one concatenation),
/// `stepConditioning(timesteps:)` (:168-213) runs every timestep as a row of
/// one pass on the device, `projectContext` (:217-245) is the bf16 context
/// embedder qmm.
public final class DirectConditionerHIP {
    public static let dim = 3072
    public static let sinDim = 256
    static let heads = ["double_stream_modulation_img.linear", "double_stream_modulation_txt.linear",
                        "single_stream_modulation.linear", "norm_out.linear"]

    public let ctx: HIPContext
    let timeL1, timeL2, modHeads, contextEmb: ProjectionQ
    let chain: OpaquePointer

    public init(transformerDirectory: String, context: HIPContext? = nil) throws {
        ctx = try context ?? HIPContext()
        let st = try SafetensorsHIP(directory: transformerDirectory)
        timeL1 = try ProjectionQ(ctx, st, "time_guidance_embed.linear_1", dtype: IMQ_F32)
        timeL2 = try ProjectionQ(ctx, st, "time_guidance_embed.linear_2", dtype: IMQ_F32)
        modHeads = try ProjectionQ(ctx, st, prefixes: Self.heads, dtype: IMQ_F32)
        contextEmb = try ProjectionQ(ctx, st, "context_embedder", dtype: IMQ_BF16)
        var a = timeL1.q, b = timeL2.q, c = modHeads.q
        var h: OpaquePointer?
        try ctx.check(imq_cond_create(ctx.ctx, &a, &b, &c, &h))
        chain = h!
    }

    deinit { imq_cond_destroy(chain) }

    /// `sinusoid(_:)` (:152-166): [cos | sin] of t * expf(-logf(10000) i / 128).
    public static func sinusoid(_ t: Float) -> [Float] {
        var out = [Float](repeating: 0, count: sinDim)
        var tt = t
        _ = out.withUnsafeMutableBufferPointer { imq_cond_sinusoid(&tt, 1, Int32(sinDim), $0.baseAddress) }
        return out
    }

    public func stepConditioning(timesteps: [Float]) throws -> [StepConditioningHIP] {
        let d = Self.dim
        let count = timesteps.count
        guard count > 0 else { return [] }
        let nHeads = modHeads.n
        let temb = try DeviceBuffer(ctx, bytes: count * d * 4)
        let heads = try DeviceBuffer(ctx, bytes: count * nHeads * 4)
        try timesteps.withUnsafeBufferPointer { t in
            try ctx.check(imq_cond_step_conditioning(
                chain, t.baseAddress, Int32(count), temb.ptr.assumingMemoryBound(to: Float.self),
                heads.ptr.assumingMemoryBound(to: Float.self), ctx.stream))
        }
        let tv = try temb.download(Float.self, count: count * d)
        let hv = try heads.download(Float.self, count: count * nHeads)
        return (0 ..< count).map { i in
            let row = Array(hv[i * nHeads ..< (i + 1) * nHeads])
            func slice(_ j: Int) -> [Float] { Array(row[j * d ..< (j + 1) * d]) }
            func triple(_ j: Int) -> ([Float], [Float], [Float]) { (slice(j), slice(j + 1), slice(j + 2)) }
            return StepConditioningHIP(
                temb: Array(tv[i * d ..< (i + 1) * d]),
                doubleImg: [triple(0), triple(3)], doubleTxt: [triple(6), triple(9)],
                single: triple(12), outScale: slice(15), outShift: slice(16))
        }
    }

    /// `projectContext`: [L, 7680] bf16 prompt embeddings (device) -> [L, dim]
    /// bf16 on the bf16 qmm (the reference widens it to f32 on the host).
    public func projectContext(embeds: DeviceBuffer, length: Int) throws -> DeviceBuffer {
        let y = try DeviceBuffer(ctx, bytes: length * Self.dim * 2)
        try QuantizedLinearHIP(ctx, contextEmb).qmm(x: embeds.ptr, y: y.ptr, m: length)
        try ctx.sync()
        return y
    }
}
