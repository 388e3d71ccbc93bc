// swift-tools-version:5.9
// The Swift call surface of libimq (the MI355X quantized-linear engine):
// `ImarelloHIP` mirrors the reference's direct-engine classes over the C ABI
// of include/*.h; `ImarelloHIPAdapter` is the PackedLatentDenoising conformance,
// built inside the reference's package (it imports MLX and ImarelloRuntime).
// Build libimq.so first (python -m aestrix_amd.build) and point IMQ_LIB_DIR at
// aestrix_amd/.
import PackageDescription
import Foundation

let libDir = ProcessInfo.processInfo.environment["IMQ_LIB_DIR"] ?? "../aestrix_amd"

let package = Package(
    name: "ImarelloHIP",
    products: [
        .library(name: "ImarelloHIP", targets: ["ImarelloHIP"]),
    ],
    targets: [
        .systemLibrary(name: "CImq", path: "Sources/CImq"),
        .target(
            name: "ImarelloHIP",
            dependencies: ["CImq"],
            path: "Sources/ImarelloHIP",
            linkerSettings: [.unsafeFlags(["-L\(libDir)", "-L/opt/rocm/lib",
                                           "-Xlinker", "-rpath", "-Xlinker", libDir])]),
    ]
)
