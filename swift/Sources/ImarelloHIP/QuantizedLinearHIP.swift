import CImq

/// The quantized-linear operator surface over the C ABI of include/imq.h:
/// `DirectDiTStep.qmm` (Sources/ImarelloDirect/DirectDiTStep.swift:374-406),
/// `AttentionUtils.applyLinear` / `applyLinearCore` with its f16 sandwich and
/// S4 options (Sources/ImarelloDiT/AttentionUtils.swift:140-230), and the glue
/// kernels the reference runs after a qmm, fused into it.  Every call is
/// asynchronous on the context's stream; pointers are device addresses.
public struct QuantizedLinearHIP {
    public let ctx: HIPContext
    public let proj: ProjectionQ
    public var dtype: imq_dtype { proj.q.dtype }

    public init(_ ctx: HIPContext, _ proj: ProjectionQ) {
        self.ctx = ctx
        self.proj = proj
    }

    /// `qmm(_:x:xOff:y:yOff:m:)`: y rows = x rows . deq(W)^T through the regime
    /// dispatcher; the byte offsets of the reference's `setBuffer(_:offset:)`
    /// are pointer offsets here.
    public func qmm(x: UnsafeRawPointer, y: UnsafeMutableRawPointer, m: Int) throws {
        let q = proj.q
        try ctx.check(imq_qmm_t(ctx.ctx, q.w, q.scales, q.biases, x, y, q.k, q.n, Int32(m), 64, 4,
                                q.dtype, ctx.stream))
    }

    /// `applyLinearCore` with `linearF16` on: x (f32 [m, K]) / scale to f16, the
    /// f16 qmm and the rescale, into y (f32, or f16 with `outputF16`).  With
    /// `dynamicTarget` the scale is `max(amax|x| / target, 1)` computed on the
    /// device (`linearDynamicScale`); `scratch` holds the f16 input (m K halves)
    /// and `scaleBuf` one float.
    public func applyLinear(x: UnsafeRawPointer, y: UnsafeMutableRawPointer, m: Int,
                            scratch: DeviceBuffer, scaleBuf: DeviceBuffer? = nil,
                            scale: Float = 16, outputF16: Bool = false,
                            dynamicTarget: Float? = nil) throws {
        let q = proj.q
        guard q.dtype == IMQ_F16 else { throw HIPError.shape("the f16 sandwich needs f16 scales") }
        let count = m * Int(q.k)
        guard scratch.bytes >= count * 2 else { throw HIPError.shape("scratch holds \(scratch.bytes) bytes") }
        var scaleDev: UnsafeMutablePointer<Float>? = nil
        if let target = dynamicTarget {
            guard let sb = scaleBuf else { throw HIPError.shape("the dynamic scale needs scaleBuf") }
            scaleDev = sb.ptr.assumingMemoryBound(to: Float.self)
            try ctx.check(imq_dynamic_scale(ctx.ctx, x.assumingMemoryBound(to: Float.self), count,
                                            target, scaleDev, ctx.stream))
        }
        try ctx.check(imq_cast_prescale_ex(ctx.ctx, x.assumingMemoryBound(to: Float.self), scratch.ptr,
                                           count, scale, scaleDev, IMQ_F16, ctx.stream))
        try ctx.check(imq_qmm_postscale_ex(ctx.ctx, q.w, q.scales, q.biases, scratch.ptr, y,
                                           outputF16 ? IMQ_F16 : IMQ_F32, q.k, q.n, Int32(m), scale,
                                           scaleDev, 64, 4, q.dtype, ctx.stream))
    }

    /// qmm then `gateAdd` / `dd_gate_add` (DirectDiTStep.swift:505-519): f32
    /// y = residual + gate * float(T(x . W^T)) * scale; y may be residual.
    public func qmmGateAdd(x: UnsafeRawPointer, residual: UnsafePointer<Float>,
                           gate: UnsafePointer<Float>, y: UnsafeMutablePointer<Float>, m: Int,
                           scale: Float = 16) throws {
        let q = proj.q
        try ctx.check(imq_qmm_gate_add(ctx.ctx, q.w, q.scales, q.biases, x, residual, gate, y, q.k,
                                       q.n, Int32(m), scale, 64, 4, q.dtype, ctx.stream))
    }

    /// qmm into the wide buffer then `swiglu` / `dd_swiglu_pitched`
    /// (DirectDiTStep.swift:521-543): y[:, j] (pitch ldy) = T(g * sigmoid(g) * u * outScale).
    public func qmmSwiGLU(x: UnsafeRawPointer, y: UnsafeMutableRawPointer, ldy: Int, m: Int,
                          width: Int, gateRow: Int, upRow: Int, inScale: Float = 16,
                          outScale: Float = 1.0 / 16) throws {
        let q = proj.q
        try ctx.check(imq_qmm_swiglu(ctx.ctx, q.w, q.scales, q.biases, x, y, Int32(ldy), q.k, q.n,
                                     Int32(m), Int32(width), Int32(gateRow), Int32(upRow), inScale,
                                     outScale, 64, 4, q.dtype, ctx.stream))
    }

    /// The text encoder's qmm + `dq_add` (DirectTEEncoder.swift:390-392):
    /// y = T(residual + T(x . W^T)); y may be residual.
    public func qmmAdd(x: UnsafeRawPointer, residual: UnsafeRawPointer, y: UnsafeMutableRawPointer,
                       m: Int) throws {
        let q = proj.q
        try ctx.check(imq_qmm_add(ctx.ctx, q.w, q.scales, q.biases, x, residual, y, q.k, q.n,
                                  Int32(m), 64, 4, q.dtype, ctx.stream))
    }
}
