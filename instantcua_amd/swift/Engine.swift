// Swift `Engine` over the MI355X C ABI (include/icua.h): the drop-in replacement for
// Sources/Engine/Engine.swift's Metal engine.  Same public surface:
// init(modelPath:maxContext:maxPass:maxSteps:copyWeights:pinMemory:), eos, usePrefixCache,
// useVisionDeltaCache, lastTiming, format/maxContext/maxPass/maxSteps, logits, poolerBuf,
// deepstackBufs, prepareMRoPE(visOffset:llmH:llmW:) and
// generateVision(rgbBytes:width:height:tokens:maxNewTokens:writeFirstLogits:).  The forced syntax
// pairs and the ")" stop of the reference's commit kernel (Shaders.swift:1543-1560) are on, as
// they always are in the reference; useGrammarPairs turns them off.
// Errors surface as EngineError (Sources/Engine/ModelFile.swift:158-161).  The C header's
// anonymous enum constants import into Swift as Int.
//
// Built only where a Swift toolchain exists (add a SwiftPM system-library target whose
// module map is CICUA/module.modulemap and link libicua.so).
import CICUA
import Foundation

public struct EngineError: Error, CustomStringConvertible {
    public let description: String
    public init(_ d: String) { description = d }
}

@inline(__always) private func check(_ rc: Int32) throws {
    if rc != 0 { throw EngineError(String(cString: icua_last_error())) }
}

public enum WeightFormat: UInt32 { case f16 = 0, q8 = 1, q4 = 2 }

/// Host copy of one of the engine's device buffers with the MTLBuffer-style `contents()` that the
/// reference's callers read (main.swift:161-169): every call copies the engine's current data
/// into host memory owned by this object and returns it.
public final class HostBuffer {
    public let length: Int
    private let storage: UnsafeMutableRawPointer
    private let fill: (UnsafeMutableRawPointer, Int) -> Void
    init(length: Int, fill: @escaping (UnsafeMutableRawPointer, Int) -> Void) {
        self.length = length
        self.storage = UnsafeMutableRawPointer.allocate(byteCount: max(length, 16), alignment: 64)
        self.storage.initializeMemory(as: UInt8.self, repeating: 0, count: max(length, 16))
        self.fill = fill
    }
    deinit { storage.deallocate() }
    public func contents() -> UnsafeMutableRawPointer {
        fill(storage, length)
        return storage
    }
}

public final class Engine {
    private let handle: OpaquePointer
    public let format: WeightFormat
    public let maxContext: Int
    public let maxPass: Int
    public let maxSteps: Int

    public var eos: (Int32, Int32) = (151645, 151643) {
        didSet { _ = icua_set_eos(handle, eos.0, eos.1) }
    }
    public var usePrefixCache: Bool = true { didSet { applyFlags() } }
    public var useGrammarPairs: Bool = true { didSet { applyFlags() } }
    public var useVisionDeltaCache: Bool = true { didSet { applyFlags() } }
    private var writeFirstLogits = false
    /// The engine's message for the last generate / generateVision call that failed (nil after a
    /// call that succeeded).  Those calls keep the reference's non-throwing signature and return
    /// an empty array on failure; this tells an empty answer from an error, e.g. "persistent
    /// decode kernel: a synchronisation wait timed out".
    public private(set) var lastError: String?

    public struct Timing {
        public var visionMs = 0.0, prefillMs = 0.0, decodeMs = 0.0, totalMs = 0.0
        public var prefillTokens = 0, generatedTokens = 0
    }
    public var lastTiming: Timing {
        var t = icua_timing_t()
        _ = icua_timing(handle, &t)
        return Timing(visionMs: t.vision_ms, prefillMs: t.prefill_ms, decodeMs: t.decode_ms, totalMs: t.total_ms,
                      prefillTokens: Int(t.prefill_tokens), generatedTokens: Int(t.generated_tokens))
    }

    /// First-token logits of the last generate call made with writeFirstLogits (Engine.swift:25).
    public private(set) lazy var logits = HostBuffer(length: 151_936 * 4) { [unowned self] p, _ in
        _ = icua_logits(self.handle, p.assumingMemoryBound(to: Float.self), 1)
    }
    /// Visual rows of the last frame: pooler [nVis][2048] float (Engine.swift:20).
    public private(set) lazy var poolerBuf = HostBuffer(length: 256 * 2048 * 4) { [unowned self] p, n in
        self.readVisual(Int32(ICUA_BUF_POOLER), p, n)
    }
    /// The three DeepStack sets of the last frame, [nVis][2048] float each (Engine.swift:21).
    public private(set) lazy var deepstackBufs: [HostBuffer] = (0..<3).map { i in
        HostBuffer(length: 256 * 2048 * 4) { [unowned self] p, n in
            self.readVisual(Int32(ICUA_BUF_DEEPSTACK0) + Int32(i), p, n)
        }
    }

    /// `copyWeights` and `pinMemory` are accepted for source compatibility with the reference's
    /// initializer and have no effect here: the engine always copies the weights into GPU memory
    /// (repacked into matrix-core tiles) while it loads, and releases the file mapping before this
    /// initializer returns, so there is neither a no-copy mode nor host memory to pin.
    public init(modelPath: String, maxContext: Int = 2048, maxPass: Int = 512, maxSteps: Int = 256,
                copyWeights: Bool = false, pinMemory: Bool = true) throws {
        var h: OpaquePointer?
        let flags = UInt32(ICUA_FLAG_PREFIX_CACHE) | UInt32(ICUA_FLAG_GRAMMAR_PAIRS) |
            UInt32(ICUA_FLAG_VISION_DELTA_CACHE)
        try check(icua_engine_create(modelPath, Int32(maxContext), Int32(maxPass), Int32(maxSteps), flags, &h))
        handle = h!
        var info = icua_info_t()
        try check(icua_engine_info(handle, &info))
        format = WeightFormat(rawValue: UInt32(info.format)) ?? .q4
        self.maxContext = Int(info.max_context)
        self.maxPass = Int(info.max_pass)
        self.maxSteps = Int(info.max_steps)
    }

    deinit { icua_engine_destroy(handle) }

    private func applyFlags() {
        var f: UInt32 = 0
        if usePrefixCache { f |= UInt32(ICUA_FLAG_PREFIX_CACHE) }
        if useGrammarPairs { f |= UInt32(ICUA_FLAG_GRAMMAR_PAIRS) }
        if useVisionDeltaCache { f |= UInt32(ICUA_FLAG_VISION_DELTA_CACHE) }
        if writeFirstLogits { f |= UInt32(ICUA_FLAG_FIRST_LOGITS) }
        _ = icua_set_flags(handle, f)
    }

    private func readVisual(_ which: Int32, _ p: UnsafeMutableRawPointer, _ cap: Int) {
        var info = icua_info_t()
        guard icua_engine_info(handle, &info) == 0 else { return }
        let bytes = min(Int(info.visual_rows) * 2048 * 4, cap)
        if bytes > 0 { _ = icua_read_buffer(handle, which, p, bytes) }
    }

    public func prepareMRoPE(visOffset: Int, llmH: Int, llmW: Int) {
        _ = icua_prepare_mrope(handle, Int32(visOffset), Int32(llmH), Int32(llmW))
    }

    /// Visual embeddings [nVis][2048] and the three DeepStack sets, when they come from outside
    /// the engine's vision tower.
    public func setVisual(pooler: [Float], deepstack: [[Float]]?, nVis: Int) throws {
        try pooler.withUnsafeBufferPointer { p in
            if let ds = deepstack {
                try ds[0].withUnsafeBufferPointer { d0 in
                    try ds[1].withUnsafeBufferPointer { d1 in
                        try ds[2].withUnsafeBufferPointer { d2 in
                            var ptrs: [UnsafePointer<Float>?] = [d0.baseAddress, d1.baseAddress, d2.baseAddress]
                            try check(icua_set_visual(handle, p.baseAddress, &ptrs, Int32(nVis)))
                        }
                    }
                }
            } else {
                try check(icua_set_visual(handle, p.baseAddress, nil, Int32(nVis)))
            }
        }
    }

    /// Prefill + GPU-resident greedy decode on visual rows from setVisual (generateVision after
    /// its vision encoder); returns the tokens before EOS.
    public func generate(tokens: [Int32], maxNewTokens: Int = 64, writeFirstLogits: Bool = false) -> [Int32] {
        let visOffset = tokens.firstIndex(of: 151655) ?? -1
        var out = [Int32](repeating: 0, count: max(maxNewTokens, 1) + 4)
        var n: Int32 = 0
        self.writeFirstLogits = writeFirstLogits
        applyFlags()
        defer { self.writeFirstLogits = false; applyFlags() }
        let rc = tokens.withUnsafeBufferPointer { t in
            icua_generate(handle, t.baseAddress, Int32(tokens.count), Int32(visOffset), Int32(maxNewTokens), &out, &n)
        }
        lastError = rc == 0 ? nil : String(cString: icua_last_error())
        return rc == 0 ? Array(out[0..<Int(n)]) : []
    }

    /// generateVision (Engine.swift:696-827) on an RGB8 frame [height][width][3]: vision tower
    /// (skipped on an identical frame when useVisionDeltaCache), prefill, greedy decode; with
    /// writeFirstLogits the first token's logits stay readable through `logits`.
    public func generateVision(rgbBytes: UnsafeRawPointer, width: Int = 640, height: Int = 384,
                               tokens: [Int32], maxNewTokens: Int = 64, writeFirstLogits: Bool = false) -> [Int32] {
        var out = [Int32](repeating: 0, count: max(maxNewTokens, 1) + 4)
        var n: Int32 = 0
        self.writeFirstLogits = writeFirstLogits
        applyFlags()
        defer { self.writeFirstLogits = false; applyFlags() }
        let rc = tokens.withUnsafeBufferPointer { t in
            icua_generate_vision(handle, rgbBytes.assumingMemoryBound(to: UInt8.self), Int32(width), Int32(height),
                                 t.baseAddress, Int32(tokens.count), Int32(maxNewTokens), &out, &n)
        }
        lastError = rc == 0 ? nil : String(cString: icua_last_error())
        return rc == 0 ? Array(out[0..<Int(n)]) : []
    }

    /// Speculative verify of up to 8 draft tokens; per-row greedy tokens.
    public func verify(draft: [Int32]) throws -> [Int32] {
        var out = [Int32](repeating: 0, count: draft.count)
        try draft.withUnsafeBufferPointer { d in
            try check(icua_verify(handle, d.baseAddress, Int32(draft.count), &out, nil))
        }
        return out
    }
}
