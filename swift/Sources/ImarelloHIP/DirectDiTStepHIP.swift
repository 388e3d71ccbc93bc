import CImq

/// The `DirectDiTStep` call surface (Sources/ImarelloDirect/DirectDiTStep.swift) over
/// include/imq_step.h: `init(lImg:)` (:74), `loadBlocks(arrays:nDouble:nSingle:)`
/// (:294), `loadHead(arrays:)` (:844), `setStepConditioning` (:887),
/// `encodeDenoiseStep(latIn:latOut:e0:head:dt:)` (:908) and `upload(_:_:)` (:135).
/// The step is one HIP graph launch (captured on the first denoise call) instead
/// of ~25 command encoders; the one blocking wait per step stays.  Attention,
/// RoPE, the per-head norms and the LayerNorm modulation are not on the
/// quantized-linear path and are not in the graph (include/imq_step.h says
/// what stands in for them).
public final class DirectDiTStepHIP {
    public static let dim = 3072
    public static let ffInner = 9216
    public static let lTxt = 512
    public static let channels = 128

    public let ctx: HIPContext
    public let lImg: Int
    var projections: [ProjectionQ] = []
    var step: OpaquePointer?
    var nDouble = 0, nSingle = 0

    /// The head's projections and the persistent latent ping-pong
    /// (`Head`, DirectDiTStep.swift:858-883).
    public final class Head {
        public let xEmb: ProjectionQ
        public let projOut: ProjectionQ
        public let latA: DeviceBuffer
        public let latB: DeviceBuffer
        init(xEmb: ProjectionQ, projOut: ProjectionQ, latA: DeviceBuffer, latB: DeviceBuffer) {
            self.xEmb = xEmb
            self.projOut = projOut
            self.latA = latA
            self.latB = latB
        }
    }

    public init(lImg: Int, context: HIPContext? = nil) throws {
        self.lImg = lImg
        ctx = try context ?? HIPContext()
    }

    deinit {
        if let s = step { imq_dit_step_destroy(s) }
    }

    /// `upload(_:_:)`: a device copy of host floats.
    public func upload(_ values: [Float]) throws -> DeviceBuffer {
        try DeviceBuffer(ctx, copying: values)
    }

    /// `loadBlocks`: every block projection from the shards, scales and biases
    /// cast to f16 (the reference's `sub()` precast, :296-307), in the order of
    /// `DoubleWeights` (:310-323) and `SingleWeights` (:328-333); then the plan.
    public func loadBlocks(weights st: SafetensorsHIP, nDouble: Int, nSingle: Int) throws {
        let double = ["attn.to_q", "attn.to_k", "attn.to_v", "attn.add_q_proj", "attn.add_k_proj",
                      "attn.add_v_proj", "attn.to_out", "attn.to_add_out", "ff.linear_in",
                      "ff.linear_out", "ff_context.linear_in", "ff_context.linear_out"]
        let single = ["attn.to_qkv_mlp_proj", "attn.to_out"]
        var loaded: [ProjectionQ] = []
        for i in 0 ..< nDouble {
            for name in double {
                loaded.append(try ProjectionQ(ctx, st, "transformer_blocks.\(i).\(name)", dtype: IMQ_F16))
            }
        }
        for i in 0 ..< nSingle {
            for name in single {
                loaded.append(try ProjectionQ(ctx, st, "single_transformer_blocks.\(i).\(name)",
                                              dtype: IMQ_F16))
            }
        }
        var dims = imq_dit_dims(l_img: Int32(lImg), l_txt: Int32(Self.lTxt), dim: Int32(Self.dim),
                                ff_inner: Int32(Self.ffInner), n_double: Int32(nDouble),
                                n_single: Int32(nSingle))
        var ws = loaded.map { $0.q }
        var s: OpaquePointer?
        try ctx.check(imq_dit_step_create(ctx.ctx, &dims, &ws, Int32(ws.count), IMQ_F16, &s))
        if let old = step { imq_dit_step_destroy(old) }
        step = s
        projections = loaded
        self.nDouble = nDouble
        self.nSingle = nSingle
    }

    /// `loadHead`: x_embedder [dim, 128] and proj_out [128, dim], f16
    /// parameters, and the latent ping-pong buffers (f32 [lImg, 128] each).
    public func loadHead(weights st: SafetensorsHIP) throws -> Head {
        guard let s = step else { throw HIPError.shape("loadBlocks first") }
        let xEmb = try ProjectionQ(ctx, st, "x_embedder", dtype: IMQ_F16)
        let projOut = try ProjectionQ(ctx, st, "proj_out", dtype: IMQ_F16)
        var a = xEmb.q, b = projOut.q
        try ctx.check(imq_dit_step_set_head(s, &a, &b))
        let bytes = lImg * Self.channels * 4
        return Head(xEmb: xEmb, projOut: projOut, latA: try DeviceBuffer(ctx, bytes: bytes),
                    latB: try DeviceBuffer(ctx, bytes: bytes))
    }

    /// `setStepConditioning` for the parts on the quantized-linear path: the
    /// RMSNorm weight [dim] and the gated-residual gates.  The reference's
    /// modulation is shared by the blocks of a kind (one img / txt triple pair
    /// for every double block, one triple for every single block); each
    /// block's gates are taken from it: img attention, txt attention, img MLP,
    /// txt MLP per double block, then one per single block.
    public func setStepConditioning(_ sc: StepConditioningHIP, normWeight: [Float]? = nil) throws {
        guard let s = step else { throw HIPError.shape("loadBlocks first") }
        var gates: [Float] = []
        gates.reserveCapacity((4 * nDouble + nSingle) * Self.dim)
        for _ in 0 ..< nDouble {
            gates += sc.doubleImg[0].2
            gates += sc.doubleTxt[0].2
            gates += sc.doubleImg[1].2
            gates += sc.doubleTxt[1].2
        }
        for _ in 0 ..< nSingle { gates += sc.single.2 }
        let g = try DeviceBuffer(ctx, copying: gates)
        let w = try normWeight.map { try DeviceBuffer(ctx, copying: $0) }
        try ctx.check(imq_dit_step_set_conditioning(
            s, w?.ptr.assumingMemoryBound(to: Float.self), g.ptr.assumingMemoryBound(to: Float.self),
            ctx.stream))
        try ctx.sync()  // the staging buffers above are released on return
    }

    /// `encodeDenoiseStep`: x_embedder sandwich -> blocks -> head norm ÷ 16 ->
    /// proj_out -> Euler (latOut = latIn + pred * dt), one graph launch and one
    /// blocking wait.  latIn / latOut f32 [lImg, 128], e0 f32 [512, dim].
    public func encodeDenoiseStep(latIn: DeviceBuffer, latOut: DeviceBuffer, e0: DeviceBuffer,
                                  head: Head, dt: Float) throws {
        guard let s = step else { throw HIPError.shape("loadBlocks first") }
        try ctx.check(imq_dit_step_denoise(s, latIn.ptr.assumingMemoryBound(to: Float.self),
                                           e0.ptr.assumingMemoryBound(to: Float.self),
                                           latOut.ptr.assumingMemoryBound(to: Float.self), dt, 1,
                                           ctx.stream))
        try ctx.sync()
    }

    /// Kernel launches of the last step encoded.
    public var launches: Int { step.map { Int(imq_dit_step_launches($0)) } ?? 0 }
}
