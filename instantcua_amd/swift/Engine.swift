// Swift `Engine` over the MI355X C ABI (include/icua.h): the drop-in replacement for
// Sources/Engine/Engine.swift's Metal engine.  Same public surface for the decoder path:
// init(modelPath:maxContext:maxPass:maxSteps:copyWeights:pinMemory:), eos, usePrefixCache,
// lastTiming, format/maxContext/maxPass/maxSteps, prepareMRoPE(visOffset:llmH:llmW:),
// generateVision(...) minus the vision encoder (the caller passes pooler/DeepStack features).
// Errors surface as EngineError (Sources/Engine/ModelFile.swift:158-161).
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
    public var useGrammarPairs: Bool = false { didSet { applyFlags() } }
    public var useVisionDeltaCache: Bool = true { didSet { applyFlags() } }

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

    public init(modelPath: String, maxContext: Int = 2048, maxPass: Int = 512, maxSteps: Int = 256,
                copyWeights: Bool = false, pinMemory: Bool = true) throws {
        var h: OpaquePointer?
        try check(icua_engine_create(modelPath, Int32(maxContext), Int32(maxPass), Int32(maxSteps),
                                     UInt32(ICUA_FLAG_PREFIX_CACHE.rawValue), &h))
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
        if usePrefixCache { f |= UInt32(ICUA_FLAG_PREFIX_CACHE.rawValue) }
        if useGrammarPairs { f |= UInt32(ICUA_FLAG_GRAMMAR_PAIRS.rawValue) }
        if useVisionDeltaCache { f |= UInt32(ICUA_FLAG_VISION_DELTA_CACHE.rawValue) }
        _ = icua_set_flags(handle, f)
    }

    public func prepareMRoPE(visOffset: Int, llmH: Int, llmW: Int) {
        _ = icua_prepare_mrope(handle, Int32(visOffset), Int32(llmH), Int32(llmW))
    }

    /// Visual embeddings [nVis][2048] and the three DeepStack sets (the ViT's outputs).
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

    /// generateVision (Engine.swift:696-827) after the vision encoder: prefill + GPU-resident
    /// greedy decode; returns the tokens before EOS.
    public func generate(tokens: [Int32], maxNewTokens: Int = 64) -> [Int32] {
        let visOffset = tokens.firstIndex(of: 151655) ?? -1
        var out = [Int32](repeating: 0, count: max(maxNewTokens, 1) + 4)
        var n: Int32 = 0
        let rc = tokens.withUnsafeBufferPointer { t in
            icua_generate(handle, t.baseAddress, Int32(tokens.count), Int32(visOffset), Int32(maxNewTokens), &out, &n)
        }
        return rc == 0 ? Array(out[0..<Int(n)]) : []
    }

    /// generateVision (Engine.swift:696-827) on an RGB8 frame [height][width][3]: vision tower
    /// (skipped on an identical frame when useVisionDeltaCache), prefill, greedy decode.
    public func generateVision(rgbBytes: UnsafeRawPointer, width: Int = 640, height: Int = 384,
                               tokens: [Int32], maxNewTokens: Int = 64) -> [Int32] {
        var out = [Int32](repeating: 0, count: max(maxNewTokens, 1) + 4)
        var n: Int32 = 0
        let rc = tokens.withUnsafeBufferPointer { t in
            icua_generate_vision(handle, rgbBytes.assumingMemoryBound(to: UInt8.self), Int32(width), Int32(height),
                                 t.baseAddress, Int32(tokens.count), Int32(maxNewTokens), &out, &n)
        }
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
