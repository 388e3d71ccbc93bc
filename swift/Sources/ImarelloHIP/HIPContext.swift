import CImq
import Glibc

/// Errors of the C ABI: the status code (`imq_status`) and the context's
/// last error text.  The reference throws `SpikeError.missingTensor` /
/// `.metal(String)` (Sources/ImarelloDirect/DirectQmmSpike.swift:17-19); a
/// missing tensor arrives here as `IMQ_EINVAL` with the tensor's name in the text.
public enum HIPError: Error, CustomStringConvertible {
    case status(Int32, String)
    case shape(String)

    public var description: String {
        switch self {
        case .status(let s, let m): return "imq status \(s): \(m)"
        case .shape(let m): return "shape: \(m)"
        }
    }
}

@inline(__always)
func imqCheck(_ status: Int32, _ ctx: OpaquePointer?) throws {
    guard status == Int32(IMQ_OK.rawValue) else {
        let text = imq_last_error(ctx).map { String(cString: $0) } ?? ""
        throw HIPError.status(status, text)
    }
}

/// The device, its context and one stream: the reference's
/// `MTLCreateSystemDefaultDevice` + command queue (DirectDiTStep.swift:74-80).
public final class HIPContext {
    public let ctx: OpaquePointer
    public let stream: UnsafeMutableRawPointer?
    public let device: Int32

    public init(device: Int32 = 0) throws {
        var c: OpaquePointer?
        try imqCheck(imq_create(device, &c), nil)
        ctx = c!
        var s: imq_stream?
        do {
            try imqCheck(imq_stream_create(ctx, &s), ctx)
        } catch {
            imq_destroy(ctx)
            throw error
        }
        stream = s
        self.device = device
    }

    deinit {
        imq_stream_destroy(ctx, stream)
        imq_destroy(ctx)
    }

    /// The one blocking call: `cb.commit(); cb.waitUntilCompleted()` plus the
    /// error check (DirectDiTStep.swift:968-970).
    public func sync() throws {
        try imqCheck(imq_stream_sync(ctx, stream), ctx)
    }

    public func check(_ status: Int32) throws { try imqCheck(status, ctx) }
}

/// Device memory (the MTLBuffer counterpart): an owned device allocation.
public final class DeviceBuffer {
    public let ptr: UnsafeMutableRawPointer
    public let bytes: Int
    let owner: HIPContext

    public init(_ owner: HIPContext, bytes: Int) throws {
        var p: UnsafeMutableRawPointer?
        try owner.check(imq_malloc(owner.ctx, bytes, &p))
        ptr = p!
        self.bytes = bytes
        self.owner = owner
    }

    /// `upload(_:_:)` (DirectDiTStep.swift:135-145): a device copy of host values.
    public convenience init<T>(_ owner: HIPContext, copying values: [T]) throws {
        try self.init(owner, bytes: max(1, values.count * MemoryLayout<T>.stride))
        try upload(values)
    }

    deinit { imq_free(owner.ctx, ptr) }

    /// Host values into the buffer (asynchronous on the context's stream; the
    /// host array is read before the call returns).
    public func upload<T>(_ values: [T], byteOffset: Int = 0) throws {
        let n = values.count * MemoryLayout<T>.stride
        guard byteOffset + n <= bytes else { throw HIPError.shape("upload of \(n) bytes past \(bytes)") }
        try values.withUnsafeBytes { raw in
            try owner.check(imq_memcpy_h2d(owner.ctx, ptr + byteOffset, raw.baseAddress, n,
                                           owner.stream))
        }
        try owner.sync()
    }

    /// The buffer's first `count` values of T (waits for the stream).
    public func download<T>(_ type: T.Type, count: Int, byteOffset: Int = 0) throws -> [T] {
        let n = count * MemoryLayout<T>.stride
        guard byteOffset + n <= bytes else { throw HIPError.shape("download of \(n) bytes past \(bytes)") }
        var out = [T](unsafeUninitializedCapacity: count) { _, initialized in initialized = count }
        try out.withUnsafeMutableBytes { raw in
            try owner.check(imq_memcpy_d2h(owner.ctx, raw.baseAddress, ptr + byteOffset, n,
                                           owner.stream))
        }
        try owner.sync()
        return out
    }

    /// A device address `byteOffset` bytes in (the reference's
    /// `setBuffer(_:offset:)` row halves, DirectDiTStep.swift:576-579).
    public func at(_ byteOffset: Int) -> UnsafeMutableRawPointer { ptr + byteOffset }
}

/// An opened set of safetensors shards (`SafetensorsLoader.shardFileNames` +
/// `loadMergedArrays`, Sources/ImarelloWeights/SafetensorsLoader.swift:6-25),
/// memory-mapped; tensors are uploaded straight from the mapping.
public final class SafetensorsHIP {
    public let handle: OpaquePointer

    public init(directory: String) throws {
        var h: OpaquePointer?
        let rc = imq_st_open_dir(directory, &h)
        guard rc == Int32(IMQ_OK.rawValue), let opened = h else {
            throw HIPError.status(rc, imq_st_last_error(h).map { String(cString: $0) } ?? directory)
        }
        handle = opened
    }

    deinit { imq_st_close(handle) }

    public func contains(_ name: String) -> Bool {
        var info = imq_st_info()
        return imq_st_find(handle, name, &info) == Int32(IMQ_OK.rawValue)
    }

    /// A tensor converted to f32 on the device (norm weights and the like).
    public func uploadF32(_ ctx: HIPContext, _ name: String, count: Int) throws -> DeviceBuffer {
        let buf = try DeviceBuffer(ctx, bytes: count * 4)
        try ctx.check(imq_st_upload(ctx.ctx, handle, name, Int32(IMQ_ST_F32.rawValue), buf.ptr,
                                    count * 4, ctx.stream))
        return buf
    }
}

/// A resident packed projection, the reference's `Q(w:s:b:n:k:)`
/// (DirectDiTStep.swift:278-284): loaded by `imq_load_qlinear(_cat)`, freed with it.
public final class ProjectionQ {
    public var q: imq_qweight
    let owner: HIPContext

    public var n: Int { Int(q.n) }
    public var k: Int { Int(q.k) }

    /// `<prefix>.weight / .scales / .biases`; several prefixes that share K are
    /// concatenated along N in order (q/k/v, gate/up, the modulation heads).
    public init(_ owner: HIPContext, _ st: SafetensorsHIP, prefixes: [String], dtype: imq_dtype) throws {
        self.owner = owner
        q = imq_qweight()
        var cstrs = prefixes.map { strdup($0) }
        defer { cstrs.forEach { free($0) } }
        let rc = cstrs.withUnsafeMutableBufferPointer { p -> Int32 in
            p.baseAddress!.withMemoryRebound(to: UnsafePointer<CChar>?.self, capacity: p.count) {
                imq_load_qlinear_cat(owner.ctx, st.handle, $0, Int32(p.count), dtype, &q, owner.stream)
            }
        }
        try owner.check(rc)
    }

    public convenience init(_ owner: HIPContext, _ st: SafetensorsHIP, _ prefix: String,
                            dtype: imq_dtype) throws {
        try self.init(owner, st, prefixes: [prefix], dtype: dtype)
    }

    deinit { imq_qweight_free(owner.ctx, &q) }
}
