import CImq

/// The work of a DiT step that is not quantized-linear, which the caller
/// provides between the block halves (include/imq_step.h): the LayerNorm
/// modulation `lnMod` (DirectDiTStep.swift:360-373), the per-head RMSNorm, RoPE
/// and attention (:553-567, :601-606, :612-615).  Buffers are device memory, rows =
/// tokens with the 512 text rows first, J rows in all; T is f16 (the step's
/// dtype); every call is asynchronous on the context's stream.
public protocol DiTBlockCore: AnyObject {
    /// The timestep's modulation (the shift / scale halves of the triples and
    /// norm_out's scale / shift), before the step's first `modulate`.
    func setStepConditioning(_ sc: StepConditioningHIP) throws
    /// `lnMod` of a block: `which` is "img.msa"/"txt.msa" (double, before
    /// attention), "img.mlp"/"txt.mlp" (double, before the MLPs) or "single";
    /// x f32 [J, dim] -> nx T [J, dim] (image and text rows each with their
    /// own modulation).
    func modulate(_ which: String, block: Int, x: DeviceBuffer, nx: DeviceBuffer) throws
    /// Double block attention: q, k, v T [J, dim] (projections, before the
    /// per-head norms and RoPE) -> attn T [J, dim].
    func attendDouble(block: Int, q: DeviceBuffer, k: DeviceBuffer, v: DeviceBuffer,
                      attn: DeviceBuffer) throws
    /// Single block attention: qkv T [J, 3 dim] -> columns [0, dim) of concat
    /// (T, rows of `pitch` elements; columns [dim, pitch) hold the MLP half).
    func attendSingle(block: Int, qkv: DeviceBuffer, concat: DeviceBuffer, pitch: Int) throws
    /// `lnMod` "out" of the head, divided by 16 (the f16 sandwich of proj_out):
    /// the image rows of x f32 [J, dim] -> nh T [lImg, dim].
    func modulateOut(x: DeviceBuffer, nh: DeviceBuffer) throws
}

/// The `DirectDiTStep` call surface (Sources/ImarelloDirect/DirectDiTStep.swift) over
/// include/imq_step.h: `init(lImg:)` (:74), `loadBlocks(arrays:nDouble:nSingle:)`
/// (:294), `loadHead(arrays:)` (:844), `setStepConditioning` (:887),
/// `encodeDenoiseStep(latIn:latOut:e0:head:dt:core:)` (:908) and `upload(_:_:)` (:135).
/// A denoise step runs every quantized projection through the block halves
/// of include/imq_step.h, with the caller's `DiTBlockCore` (attention, RoPE,
/// the per-head norms, the LayerNorm modulation) between them.
/// `encodeStandInStep` runs the same projections as one HIP graph launch with
/// stand-ins for that core (RMSNorm for lnMod, V for attention): the
/// quantized-linear work of a step at its real shapes, but not the model's
/// output.
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

    /// The caller's buffers of the block halves (allocated on first use).
    final class HalfBuffers {
        let x, nx, q, k, v, attn, qkv, concat, nh: DeviceBuffer
        init(_ ctx: HIPContext, joint: Int, lImg: Int) throws {
            let d = DirectDiTStepHIP.dim, f = DirectDiTStepHIP.ffInner
            x = try DeviceBuffer(ctx, bytes: joint * d * 4)
            nx = try DeviceBuffer(ctx, bytes: joint * d * 2)
            q = try DeviceBuffer(ctx, bytes: joint * d * 2)
            k = try DeviceBuffer(ctx, bytes: joint * d * 2)
            v = try DeviceBuffer(ctx, bytes: joint * d * 2)
            attn = try DeviceBuffer(ctx, bytes: joint * d * 2)
            qkv = try DeviceBuffer(ctx, bytes: joint * 3 * d * 2)
            concat = try DeviceBuffer(ctx, bytes: joint * (d + f) * 2)
            nh = try DeviceBuffer(ctx, bytes: lImg * d * 2)
        }
    }
    var halves: HalfBuffers?

    /// `encodeDenoiseStep`: x_embedder sandwich -> 5 double + 20 single blocks
    /// -> norm_out ÷ 16 -> proj_out -> Euler (latOut = latIn + pred * dt), every
    /// quantized projection through the block halves and the model's
    /// non-quantized work from `core`; one blocking wait.  latIn / latOut f32
    /// [lImg, 128], e0 f32 [512, dim].
    public func encodeDenoiseStep(latIn: DeviceBuffer, latOut: DeviceBuffer, e0: DeviceBuffer,
                                  head: Head, dt: Float, core: DiTBlockCore) throws {
        guard let s = step else { throw HIPError.shape("loadBlocks first") }
        let joint = Self.lTxt + lImg
        if halves == nil { halves = try HalfBuffers(ctx, joint: joint, lImg: lImg) }
        let b = halves!
        let xf = b.x.ptr.assumingMemoryBound(to: Float.self)
        let st = ctx.stream
        try ctx.check(imq_memcpy_d2d(ctx.ctx, b.x.ptr, e0.ptr, Self.lTxt * Self.dim * 4, st))
        try ctx.check(imq_dit_head_embed(s, latIn.ptr.assumingMemoryBound(to: Float.self), xf, st))
        for blk in 0 ..< nDouble {
            try core.modulate("img.msa", block: blk, x: b.x, nx: b.nx)
            try ctx.check(imq_dit_double_attn_in(s, Int32(blk), xf, b.nx.ptr, b.q.ptr, b.k.ptr,
                                                 b.v.ptr, st))
            try core.attendDouble(block: blk, q: b.q, k: b.k, v: b.v, attn: b.attn)
            try ctx.check(imq_dit_double_attn_out(s, Int32(blk), b.attn.ptr, xf, st))
            try core.modulate("img.mlp", block: blk, x: b.x, nx: b.nx)
            try ctx.check(imq_dit_double_mlp(s, Int32(blk), b.nx.ptr, xf, st))
        }
        for blk in 0 ..< nSingle {
            try core.modulate("single", block: blk, x: b.x, nx: b.nx)
            try ctx.check(imq_dit_single_attn_in(s, Int32(blk), xf, b.nx.ptr, b.qkv.ptr,
                                                 b.concat.ptr, st))
            try core.attendSingle(block: blk, qkv: b.qkv, concat: b.concat,
                                  pitch: Self.dim + Self.ffInner)
            try ctx.check(imq_dit_single_attn_out(s, Int32(blk), b.concat.ptr, xf, st))
        }
        try core.modulateOut(x: b.x, nh: b.nh)
        try ctx.check(imq_dit_head_out(s, xf, b.nh.ptr, latIn.ptr.assumingMemoryBound(to: Float.self),
                                       latOut.ptr.assumingMemoryBound(to: Float.self), dt, st))
        try ctx.sync()
    }

    /// The step's quantized projections with the plan's stand-ins for the
    /// non-quantized work (include/imq_step.h): one graph launch and one
    /// blocking wait, for timing and checking the projections at the real
    /// shapes.  Its output is not the model's.
    public func encodeStandInStep(latIn: DeviceBuffer, latOut: DeviceBuffer, e0: DeviceBuffer,
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
