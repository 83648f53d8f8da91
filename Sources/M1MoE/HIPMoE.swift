// The M1MoE engine's GPU back end on libm1moe_hip (MI355X), over the C ABI
// of include/m1moe_hip.h imported as the CM1MoEHIP module.
//
// HIPMoE replaces the MoE part of MetalContext (MetalContext.swift:69-185)
// and the CPU router, loadExpert, encodeExpertForward and encodeMoECombine
// of InferenceEngine.swift (:240-266, :271-280, :495-519).  HIPDecoder
// replaces InferenceEngine.forward(token:) (:125-156) at temperature 0.
//
// Not compiled in this source tree (it has no Swift toolchain); it is the
// file a maintainer adds to Sources/M1MoE of the Swift package.

import CM1MoEHIP
import Foundation

public enum HIPError: Error, CustomStringConvertible {
    case status(Int32, String)
    case missingWeight(String)

    public var description: String {
        switch self {
        case let .status(rc, msg): return "libm1moe_hip status \(rc): \(msg)"
        case let .missingWeight(key): return "missing weight \(key)"
        }
    }
}

/// Every libm1moe_hip call returns 0 or an M1MOE_ERR_* status; the message
/// of the last failure on this thread is in m1moe_last_error().
@inline(__always) func hipCheck(_ rc: Int32) throws {
    if rc != 0 { throw HIPError.status(rc, String(cString: m1moe_last_error())) }
}

/// Weight key of one layer's router, as the engine names it
/// (InferenceEngine.swift:593-598).
func hipRouterKey(_ spec: ModelSpec, _ layer: Int) -> String {
    spec.architecture == "mixtral"
        ? "model.layers.\(layer).block_sparse_moe.gate.weight"
        : "model.layers.\(layer).mlp.gate.weight"
}

public final class HIPMoE {
    /// The context: resident experts of every layer, bf16 routers, the
    /// stream the calls are ordered on, and the device error flag.
    public private(set) var ctx: m1moe_ctx_t?
    public let spec: ModelSpec
    private var dX: UnsafeMutableRawPointer?
    private var dRes: UnsafeMutableRawPointer?
    private var dOut: UnsafeMutableRawPointer?

    public init(spec: ModelSpec, device: Int32 = 0) throws {
        self.spec = spec
        var shape = m1moe_moe_shape(
            hidden: Int32(spec.hiddenDim), num_experts: Int32(spec.moe.numExperts),
            top_k: Int32(spec.moe.topK), intermediate: Int32(spec.moe.intermediateDim),
            group_size: Int32(spec.quantization.groupSize), num_layers: Int32(spec.numLayers),
            norm_topk_prob: spec.moe.normTopkProb ? 1 : 0)
        try hipCheck(m1moe_create(device, &shape, &ctx))
        let hF = UInt64(spec.hiddenDim * MemoryLayout<Float>.size)
        try hipCheck(m1moe_alloc(ctx, hF, &dX))
        try hipCheck(m1moe_alloc(ctx, hF, &dRes))
        try hipCheck(m1moe_alloc(ctx, hF, &dOut))
    }

    deinit { m1moe_destroy(ctx) }       // frees the buffers above with it

    /// Replaces the per-layer pread file descriptors and the expert cache
    /// (InferenceEngine.swift:62-77, ExpertCache.swift): the whole
    /// layer_NN.bin image goes to HBM once and stays there.
    public func uploadLayer(_ layer: Int, image: Data) throws {
        try image.withUnsafeBytes { raw in
            try hipCheck(m1moe_upload_layer_experts(ctx, Int32(layer), raw.baseAddress,
                                                    UInt64(raw.count)))
        }
    }

    /// Reads and uploads every layer_NN.bin of the model directory.
    public func uploadAllLayers(modelDir: String) throws {
        for layer in 0 ..< spec.numLayers {
            let path = (modelDir as NSString)
                .appendingPathComponent(String(format: "layer_%02d.bin", layer))
            try uploadLayer(layer, image: try Data(contentsOf: URL(fileURLWithPath: path),
                                                   options: .alwaysMapped))
        }
    }

    /// Replaces the f32 router pre-conversion (InferenceEngine.swift:99-113):
    /// the router stays bf16 in HBM.
    public func uploadRouters(_ weights: WeightStore) throws {
        for layer in 0 ..< spec.numLayers {
            let key = hipRouterKey(spec, layer)
            guard let p = weights.bf16(named: key) else { throw HIPError.missingWeight(key) }
            try hipCheck(m1moe_upload_router(ctx, Int32(layer), p,
                                             UInt64(spec.moe.numExperts * spec.hiddenDim)))
        }
    }

    /// The MoE block of runLayer (InferenceEngine.swift:240-266) from host
    /// buffers: out = residual + sum_k w_k * expert_k(x), router and top-K on
    /// the GPU.  Synchronous, like the reference's commit-and-wait.
    public func forward(layer: Int, x: UnsafePointer<Float>, residual: UnsafePointer<Float>,
                        out: UnsafeMutablePointer<Float>) throws {
        let hF = UInt64(spec.hiddenDim * MemoryLayout<Float>.size)
        try hipCheck(m1moe_copy_h2d(ctx, dX, x, hF))
        try hipCheck(m1moe_copy_h2d(ctx, dRes, residual, hF))
        try hipCheck(m1moe_moe_decode(ctx, Int32(layer), dX, Int32(M1MOE_F32),
                                      dRes?.assumingMemoryBound(to: Float.self),
                                      dOut?.assumingMemoryBound(to: Float.self), nil, nil))
        try hipCheck(m1moe_copy_d2h(ctx, out, dOut, hF))
        try hipCheck(m1moe_sync(ctx))   // reports a bad expert index from the device
    }

    /// The MoE block for T prompt tokens at once, device pointers throughout
    /// (the reference forwards a prompt token by token,
    /// Sources/bench/main.swift:139-141).  dX: T x hidden (bf16 or f32),
    /// dRes (nullable) and dOut: T x hidden f32.  Asynchronous.
    public func prefill(layer: Int, tokens: Int, dX: UnsafeRawPointer, xIsBF16: Bool,
                        dRes: UnsafePointer<Float>?, dOut: UnsafeMutablePointer<Float>) throws {
        try hipCheck(m1moe_moe_prefill(ctx, Int32(layer), Int32(tokens), dX,
                                       Int32(xIsBF16 ? M1MOE_BF16 : M1MOE_F32),
                                       dRes, dOut, nil, nil))
    }
}

/// The whole decoder step on the GPU: embedding, attention with the KV
/// cache, the MoE blocks of every layer, the final norm, the LM head and the
/// greedy argmax.  Keep the HIPMoE alive for as long as this object.
public final class HIPDecoder {
    private let moe: HIPMoE
    private var dec: m1moe_dec_t?
    private var dTok: UnsafeMutableRawPointer?
    private var dLogits: UnsafeMutableRawPointer?
    private var logits: [Float]

    /// InferenceEngine.seqPos (InferenceEngine.swift:25): the next position,
    /// read from the device (m1moe_dec_position waits for the context stream).
    public var seqPos: Int {
        var p: Int32 = 0
        return m1moe_dec_position(dec, &p) == 0 ? Int(p) : -1
    }

    public init(moe: HIPMoE, weights: WeightStore) throws {
        self.moe = moe
        self.logits = [Float](repeating: 0, count: moe.spec.vocabSize)
        let spec = moe.spec
        let att = spec.attention
        var shape = m1moe_dec_shape(
            vocab: Int32(spec.vocabSize), num_heads: Int32(att.numHeads),
            num_kv_heads: Int32(att.numKvHeads), head_dim: Int32(att.headDim),
            max_seq: Int32(att.gpuKvSeqPrealloc),
            qk_norm: spec.architecture == "olmoe" ? 1 : 0,     // InferenceEngine.swift:55
            rope_theta: att.ropeTheta, rms_eps: spec.rmsNormEps)
        try hipCheck(m1moe_dec_create(moe.ctx, &shape, &dec))

        // One upload per weight key (InferenceEngine.swift:580-599).
        func up(_ which: Int, _ layer: Int, _ key: String, _ count: Int) throws {
            guard let p = weights.bf16(named: key) else { throw HIPError.missingWeight(key) }
            try hipCheck(m1moe_dec_upload(dec, Int32(which), Int32(layer), p, UInt64(count)))
        }
        let h = spec.hiddenDim, V = spec.vocabSize
        try up(M1MOE_W_EMBED, 0, "model.embed_tokens.weight", V * h)
        try up(M1MOE_W_LM_HEAD, 0, "lm_head.weight", V * h)
        try up(M1MOE_W_FINAL_NORM, 0, "model.norm.weight", h)
        for L in 0 ..< spec.numLayers {
            let pre = "model.layers.\(L)."
            try up(M1MOE_W_IN_NORM, L, pre + "input_layernorm.weight", h)
            try up(M1MOE_W_POST_NORM, L, pre + "post_attention_layernorm.weight", h)
            try up(M1MOE_W_Q, L, pre + "self_attn.q_proj.weight", att.qDim * h)
            try up(M1MOE_W_K, L, pre + "self_attn.k_proj.weight", att.kvDim * h)
            try up(M1MOE_W_V, L, pre + "self_attn.v_proj.weight", att.kvDim * h)
            try up(M1MOE_W_O, L, pre + "self_attn.o_proj.weight", h * att.qDim)
            if spec.architecture == "olmoe" {   // the first head_dim values, as the engine reads them
                try up(M1MOE_W_Q_NORM, L, pre + "self_attn.q_norm.weight", att.headDim)
                try up(M1MOE_W_K_NORM, L, pre + "self_attn.k_norm.weight", att.headDim)
            }
        }
        try hipCheck(m1moe_alloc(moe.ctx, 16, &dTok))
        try hipCheck(m1moe_alloc(moe.ctx, UInt64(4 * V), &dLogits))
    }

    deinit { m1moe_dec_destroy(dec) }   // before the HIPMoE's context, which `moe` keeps alive

    /// InferenceEngine.forward(token:temperature:topP:) (InferenceEngine.swift:
    /// 125-156).  At temperature <= 0 the greedy token is the step's own
    /// device-side argmax: one call and one 4-byte read-back.  Otherwise the
    /// step's f32 logits are read back and sampled on the host as the
    /// reference does (sampleToken below).
    @discardableResult
    public func forward(token: UInt32, temperature: Float = 0, topP: Float = 1) throws -> UInt32 {
        var t = Int32(bitPattern: token)
        let p = dTok!.assumingMemoryBound(to: Int32.self)
        let sampled = temperature > 0
        try hipCheck(m1moe_copy_h2d(moe.ctx, dTok, &t, 4))
        try hipCheck(m1moe_dec_step(dec, p, p,
                                    sampled ? dLogits!.assumingMemoryBound(to: Float.self) : nil))
        if sampled {
            try logits.withUnsafeMutableBytes {
                try hipCheck(m1moe_copy_d2h(moe.ctx, $0.baseAddress, dLogits, UInt64($0.count)))
            }
        } else {
            try hipCheck(m1moe_copy_d2h(moe.ctx, &t, dTok, 4))
        }
        try hipCheck(m1moe_sync(moe.ctx))   // reports a token outside the vocabulary or a full cache
        if !sampled { return UInt32(bitPattern: t) }
        return logits.withUnsafeBufferPointer {
            HIPDecoder.sampleToken(logits: $0.baseAddress!, count: $0.count,
                                   temperature: temperature, topP: topP)
        }
    }

    /// sampleToken (InferenceEngine.swift:550-575) on the host, in the same
    /// f32 order: exp((l - max) / T) with a sequential sum, the nucleus in
    /// descending probability until its running sum reaches topP, then a
    /// uniform draw walked down the nucleus.  Equal probabilities keep the
    /// lower index first (the reference's sort leaves their order open).
    static func sampleToken(logits: UnsafePointer<Float>, count: Int,
                            temperature: Float, topP: Float) -> UInt32 {
        if temperature <= 0 {
            var best = 0; var bestV = logits[0]
            for i in 1 ..< count where logits[i] > bestV { bestV = logits[i]; best = i }
            return UInt32(best)
        }
        var probs = [Float](repeating: 0, count: count)
        var mx = logits[0]
        for i in 1 ..< count where logits[i] > mx { mx = logits[i] }
        var sum: Float = 0
        for i in 0 ..< count { probs[i] = expf((logits[i] - mx) / temperature); sum += probs[i] }
        let inv = 1.0 / sum
        for i in 0 ..< count { probs[i] *= inv }
        let order = probs.indices.sorted {
            probs[$0] > probs[$1] || (probs[$0] == probs[$1] && $0 < $1)
        }
        var cumul: Float = 0
        var nucleus: [Int] = []
        for idx in order {
            nucleus.append(idx); cumul += probs[idx]
            if cumul >= topP { break }
        }
        var r = Float.random(in: 0 ..< cumul)
        for idx in nucleus { r -= probs[idx]; if r <= 0 { return UInt32(idx) } }
        return UInt32(nucleus.last!)
    }

    /// The bench loop (Sources/bench/main.swift:136-163) with no host round
    /// trip per token: the prompt in one batch per layer, then `nGen` greedy
    /// steps, each feeding back the token the previous one wrote.
    public func generate(prompt: [UInt32], nGen: Int) throws -> [UInt32] {
        let n = prompt.count + nGen + 1
        var seq = prompt.map { Int32(bitPattern: $0) } + [Int32](repeating: 0, count: n - prompt.count)
        var dSeq: UnsafeMutableRawPointer?
        try hipCheck(m1moe_alloc(moe.ctx, UInt64(4 * n), &dSeq))
        defer { _ = m1moe_free(moe.ctx, dSeq) }
        let s = dSeq!.assumingMemoryBound(to: Int32.self)
        try hipCheck(m1moe_copy_h2d(moe.ctx, dSeq, &seq, UInt64(4 * n)))
        try hipCheck(m1moe_dec_reset(dec))
        try hipCheck(m1moe_dec_prefill(dec, s, Int32(prompt.count), s + prompt.count, nil))
        for i in 0 ..< nGen {
            try hipCheck(m1moe_dec_step(dec, s + prompt.count + i, s + prompt.count + i + 1, nil))
        }
        try hipCheck(m1moe_copy_d2h(moe.ctx, &seq, dSeq, UInt64(4 * n)))
        try hipCheck(m1moe_sync(moe.ctx))
        return seq[prompt.count ..< n].map { UInt32(bitPattern: $0) }
    }

    /// InferenceEngine.reset (:159-163).
    public func reset() throws { try hipCheck(m1moe_dec_reset(dec)) }
}

/// Tokenizer (Tokenizer.swift:17-229) on libm1moe_hip's host code: the same
/// init(url:), encode(_:addBOS:bos:) and decode(_:skipSpecial:), so the chat
/// and bench targets switch by changing the type they construct.
public final class HIPTokenizer {
    private var tok: m1moe_tokenizer_t?

    public init(url: URL) throws {
        try hipCheck(m1moe_tokenizer_load(url.path, &tok))
    }

    deinit { m1moe_tokenizer_free(tok) }

    public func encode(_ text: String, addBOS: Bool = true, bos: UInt32 = 1) -> [UInt32] {
        let bytes = Array(text.utf8)
        return bytes.withUnsafeBufferPointer { b -> [UInt32] in
            let p = UnsafeRawPointer(b.baseAddress)?.assumingMemoryBound(to: CChar.self)
            var n: UInt64 = 0
            guard m1moe_tokenizer_encode(tok, p, UInt64(b.count), addBOS ? 1 : 0, bos,
                                         nil, 0, &n) == 0 else { return [] }
            var ids = [UInt32](repeating: 0, count: Int(n))
            let rc = ids.withUnsafeMutableBufferPointer {
                m1moe_tokenizer_encode(tok, p, UInt64(b.count), addBOS ? 1 : 0, bos,
                                       $0.baseAddress, n, &n)
            }
            return rc == 0 ? ids : []
        }
    }

    public func decode(_ ids: [UInt32], skipSpecial: Bool = true) -> String {
        var len: UInt64 = 0
        guard m1moe_tokenizer_decode(tok, ids, UInt64(ids.count), skipSpecial ? 1 : 0,
                                     nil, 0, &len) == 0 else { return "" }
        var buf = [CChar](repeating: 0, count: Int(len) + 1)
        guard m1moe_tokenizer_decode(tok, ids, UInt64(ids.count), skipSpecial ? 1 : 0,
                                     &buf, UInt64(buf.count), &len) == 0 else { return "" }
        // the bytes are UTF-8 (the library transcodes its ISO-8859-1 fallback)
        // and may hold NULs, so they are not read as a C string
        return String(decoding: buf.prefix(Int(len)).map { UInt8(bitPattern: $0) }, as: UTF8.self)
    }
}
