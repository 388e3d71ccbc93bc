// The PackedLatentDenoising conformance over ImarelloHIP, built as a target of
// the reference's package (it needs MLX, ImarelloRuntime and ImarelloDiT):
//   .target(name: "ImarelloHIPAdapter",
//           dependencies: ["ImarelloHIP", "ImarelloRuntime", "ImarelloDiT",
//                          .product(name: "MLX", package: "mlx-swift")])
import Foundation
import MLX
import ImarelloDiT
import ImarelloHIP
import ImarelloRuntime

/// `DirectDiTPackedDenoiser` (Sources/ImarelloDirect/DirectDiTAdapter.swift:14-81) on the
/// MI355X engine: the pipeline's noise and prompt embeds in, the final packed
/// latents out, behind `PackedLatentDenoising.denoise`
/// (Sources/ImarelloRuntime/ImarelloPipeline.swift:22-28).  Every quantized
/// projection of a step runs on the engine's block halves; the step's other
/// work (LayerNorm modulation, per-head norms, RoPE, attention) is the
/// caller's `DiTBlockCore`, without which no denoiser can be made.  Everything
/// else is built inside the call and freed on return (staged residency, as the
/// reference's adapter).
public final class HIPPackedDenoiser: PackedLatentDenoising {
    let transformerDirectory: URL
    let device: Int32
    let core: DiTBlockCore

    public init(transformerDirectory: URL, core: DiTBlockCore, device: Int32 = 0) {
        self.transformerDirectory = transformerDirectory
        self.core = core
        self.device = device
    }

    public func denoise(
        noise: MLXArray, embeds: MLXArray,
        width: Int, height: Int, steps: Int,
        onStep: ((Int) throws -> Void)?
    ) throws -> MLXArray {
        let lImg = (width / 16) * (height / 16)
        let dim = DirectDiTStepHIP.dim
        let ctx = try HIPContext(device: device)

        // Context projection on the bf16 qmm, widened to f32 like the
        // reference's projectContext (DirectConditioner.swift:217-245).
        let conditioner = try DirectConditionerHIP(transformerDirectory: transformerDirectory.path,
                                                   context: ctx)
        let L = embeds.dim(1)
        let e16 = embeds.asType(.bfloat16)
        eval(e16)
        let eBits: [UInt16] = e16.asData(noCopy: false).withUnsafeBytes {
            Array($0.bindMemory(to: UInt16.self))
        }
        let projected = try conditioner.projectContext(embeds: try DeviceBuffer(ctx, copying: eBits),
                                                       length: L)
        let e0 = try projected.download(UInt16.self, count: L * dim).map {
            Float(bitPattern: UInt32($0) << 16)
        }

        let engine = try DirectDiTStepHIP(lImg: lImg, context: ctx)
        let st = try SafetensorsHIP(directory: transformerDirectory.path)
        try engine.loadBlocks(weights: st, nDouble: 5, nSingle: 20)
        let head = try engine.loadHead(weights: st)

        let scheduler = Flux2Scheduler(numInferenceSteps: steps, imageSeqLen: lImg)
        let conditioning = try conditioner.stepConditioning(timesteps: scheduler.timesteps)
        let dts: [Float] = (0 ..< scheduler.sigmas.count - 1).map {
            scheduler.sigmas[$0 + 1] - scheduler.sigmas[$0]
        }

        let e0Buf = try engine.upload(e0)
        let noise32 = noise.asType(.float32)
        eval(noise32)
        try head.latA.upload(noise32.asArray(Float.self))
        var cur = head.latA, alt = head.latB
        for step in 0 ..< steps {
            try onStep?(step)
            try engine.setStepConditioning(conditioning[step])
            try core.setStepConditioning(conditioning[step])
            try engine.encodeDenoiseStep(latIn: cur, latOut: alt, e0: e0Buf, head: head, dt: dts[step],
                                         core: core)
            swap(&cur, &alt)
        }
        let lat = try cur.download(Float.self, count: lImg * DirectDiTStepHIP.channels)
        let latents = MLXArray(lat, [1, lImg, DirectDiTStepHIP.channels])
        eval(latents)
        return latents
    }
}
