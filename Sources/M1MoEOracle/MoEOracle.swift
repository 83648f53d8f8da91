// MoEOracle.swift — scalar CPU restatement, in Swift, of the MoE-layer decode
// of koaWood/M1MoE: the Swift-side checker of HIPMoE (Sources/M1MoE/HIPMoE.swift).
//
// TEST INFRASTRUCTURE ONLY.  The hipcheck executable (Sources/hipcheck) runs
// it beside HIPMoE on seeded synthetic layers; the M1MoE library neither
// depends on it nor calls it.  Not compiled in this source tree (there is no
// Swift toolchain here): it restates, step for step and in the same f32 / f64
// order, the C oracle that the repository's tests build, pin and run
// (oracle/m1moe_oracle.c: orc_matvec4bit_lanes, orc_swiglu,
// orc_router_logits, orc_softmax, orc_select_topk, orc_combine).
//
// Semantics restated (paths in koaWood/M1MoE):
//   expert block layout     ModelSpec.swift:36-52, InferenceEngine.swift:84-97
//   4-bit dequant matvec    Shaders.metal:39-92 (matvec4bit: 64 lanes, each a
//                           strided set of packed words, then a tree sum)
//   SwiGLU                  Shaders.metal:138-149
//   router + softmax        InferenceEngine.swift:490-508; the logits are
//                           the exact bf16 x f32 products summed in f64 and
//                           rounded once to f32
//   top-K (+ renorm)        InferenceEngine.swift:510-519; descending logit,
//                           ties to the lower index
//   expert FFN              InferenceEngine.swift:401-444
//   combine + residual      Shaders.metal:360-376

import Foundation

public struct MoEOracleShape {
    public let hidden: Int
    public let numExperts: Int
    public let topK: Int
    public let intermediate: Int
    public let groupSize: Int
    public let normTopkProb: Bool

    public init(hidden: Int, numExperts: Int, topK: Int, intermediate: Int, groupSize: Int,
                normTopkProb: Bool) {
        self.hidden = hidden
        self.numExperts = numExperts
        self.topK = topK
        self.intermediate = intermediate
        self.groupSize = groupSize
        self.normTopkProb = normTopkProb
    }
}

/// Byte offsets of the nine parts of one expert block (gate, up, down: packed
/// words, bf16 scales, bf16 biases) and the block's size.
public struct MoEOracleOffsets {
    public let gateW, gateS, gateB, upW, upS, upB, downW, downS, downB, expertBytes: Int
}

public enum MoEOracle {
    public static func bf16ToFloat(_ v: UInt16) -> Float {
        Float(bitPattern: UInt32(v) << 16)
    }

    public static func offsets(_ s: MoEOracleShape) -> MoEOracleOffsets {
        let h = s.hidden, i = s.intermediate, gs = s.groupSize
        let gw = i * (h / 8) * 4       // gate / up packed words
        let gsb = i * (h / gs) * 2     // gate / up scales or biases
        let dw = h * (i / 8) * 4       // down packed words
        let dsb = h * (i / gs) * 2     // down scales or biases
        let gateS = gw, gateB = gateS + gsb, upW = gateB + gsb, upS = upW + gw
        let upB = upS + gsb, downW = upB + gsb, downS = downW + dw, downB = downS + dsb
        return MoEOracleOffsets(gateW: 0, gateS: gateS, gateB: gateB, upW: upW, upS: upS, upB: upB,
                                downW: downW, downS: downS, downB: downB,
                                expertBytes: downB + dsb)
    }

    /// Shaders.metal:39-92, lane by lane: lane l sums packed words l, l + 64,
    /// ... of the row, each nibble as fma(n, s * x, fma(b, x, acc)); the 64
    /// lane sums are then added in a tree of halving strides.
    public static func matvec4bit(w: UnsafePointer<UInt32>, s: UnsafePointer<UInt16>,
                                  b: UnsafePointer<UInt16>, x: [Float], outDim: Int,
                                  inDim: Int, groupSize: Int) -> [Float] {
        let numWords = inDim / 8, numGroups = inDim / groupSize
        var y = [Float](repeating: 0, count: outDim)
        var shared = [Float](repeating: 0, count: 64)
        for row in 0 ..< outDim {
            let wRow = w + row * numWords
            let sRow = s + row * numGroups
            let bRow = b + row * numGroups
            for lid in 0 ..< 64 {
                var acc: Float = 0
                var wi = lid
                while wi < numWords {
                    let packed = wRow[wi]
                    let g = (wi * 8) / groupSize
                    let scale = bf16ToFloat(sRow[g]), bias = bf16ToFloat(bRow[g])
                    let base = wi * 8
                    for bb in 0 ..< 8 {
                        let nib = Float((packed >> UInt32(4 * bb)) & 0xF)
                        let xv = x[base + bb]
                        acc = acc.addingProduct(bias, xv).addingProduct(nib, scale * xv)
                    }
                    wi += 64
                }
                shared[lid] = acc
            }
            var st = 32
            while st > 0 {
                for lid in 0 ..< st { shared[lid] += shared[lid + st] }
                st >>= 1
            }
            y[row] = shared[0]
        }
        return y
    }

    /// Shaders.metal:147-148: silu(gate) * up.
    public static func swiglu(gate: [Float], up: [Float]) -> [Float] {
        var act = [Float](repeating: 0, count: gate.count)
        for i in 0 ..< gate.count {
            let g = gate[i]
            act[i] = (g / (1 + exp(-g))) * up[i]
        }
        return act
    }

    /// InferenceEngine.swift:490-498: one logit per expert; bf16 (8
    /// significant bits) times f32 (24) is exact in f64, and the f64 sum is
    /// rounded once.
    public static func routerLogits(router: UnsafePointer<UInt16>, x: [Float], numExperts: Int,
                                    hidden: Int) -> [Float] {
        var logits = [Float](repeating: 0, count: numExperts)
        for e in 0 ..< numExperts {
            let row = router + e * hidden
            var acc: Double = 0
            for d in 0 ..< hidden { acc += Double(bf16ToFloat(row[d])) * Double(x[d]) }
            logits[e] = Float(acc)
        }
        return logits
    }

    /// InferenceEngine.swift:500-506.
    public static func softmax(_ logits: [Float]) -> [Float] {
        var mx = logits[0]
        for e in 1 ..< logits.count where logits[e] > mx { mx = logits[e] }
        var probs = [Float](repeating: 0, count: logits.count)
        var sum: Float = 0
        for e in 0 ..< logits.count {
            probs[e] = exp(logits[e] - mx)
            sum += probs[e]
        }
        let inv = 1 / sum
        for e in 0 ..< logits.count { probs[e] *= inv }
        return probs
    }

    /// InferenceEngine.swift:510-519: the k largest logits (the lower index
    /// first among equal ones), their probabilities as weights, renormalised
    /// over the selection in slot order when normTopkProb is set.
    public static func selectTopK(logits: [Float], probs: [Float], k: Int,
                                  normTopkProb: Bool) -> (idx: [Int], w: [Float]) {
        var taken = [Bool](repeating: false, count: logits.count)
        var idx: [Int] = []
        var w: [Float] = []
        for _ in 0 ..< k {
            var best = -1
            for e in 0 ..< logits.count where !taken[e] {
                if best < 0 || logits[e] > logits[best] { best = e }
            }
            taken[best] = true
            idx.append(best)
            w.append(probs[best])
        }
        if normTopkProb {
            var ssum: Float = 0
            for j in 0 ..< k { ssum = ssum + w[j] }
            for j in 0 ..< k { w[j] = w[j] / ssum }
        }
        return (idx, w)
    }

    /// Shaders.metal:360-376: out = residual + sum_k w_k y_k, slots in order.
    public static func combine(expertOuts: [[Float]], w: [Float], residual: [Float]?) -> [Float] {
        let h = expertOuts[0].count
        var out = [Float](repeating: 0, count: h)
        for d in 0 ..< h {
            var acc: Float = residual?[d] ?? 0
            for j in 0 ..< w.count { acc = acc.addingProduct(w[j], expertOuts[j][d]) }
            out[d] = acc
        }
        return out
    }

    /// InferenceEngine.swift:401-444: gate, up, SwiGLU, down of one expert.
    public static func expertForward(shape s: MoEOracleShape, block: UnsafeRawPointer,
                                     x: [Float]) -> [Float] {
        let o = offsets(s)
        func u32(_ off: Int) -> UnsafePointer<UInt32> {
            (block + off).assumingMemoryBound(to: UInt32.self)
        }
        func u16(_ off: Int) -> UnsafePointer<UInt16> {
            (block + off).assumingMemoryBound(to: UInt16.self)
        }
        let gate = matvec4bit(w: u32(o.gateW), s: u16(o.gateS), b: u16(o.gateB), x: x,
                              outDim: s.intermediate, inDim: s.hidden, groupSize: s.groupSize)
        let up = matvec4bit(w: u32(o.upW), s: u16(o.upS), b: u16(o.upB), x: x,
                            outDim: s.intermediate, inDim: s.hidden, groupSize: s.groupSize)
        let act = swiglu(gate: gate, up: up)
        return matvec4bit(w: u32(o.downW), s: u16(o.downS), b: u16(o.downB), x: act,
                          outDim: s.hidden, inDim: s.intermediate, groupSize: s.groupSize)
    }

    /// The MoE block (InferenceEngine.swift:240-266): router, top-K, the
    /// selected experts of the layer image (expert e at e * expertBytes) and
    /// the combine with the residual.
    public static func decode(shape s: MoEOracleShape, layerImage: UnsafeRawPointer,
                              router: UnsafePointer<UInt16>, x: [Float],
                              residual: [Float]?) -> (out: [Float], idx: [Int], w: [Float]) {
        let logits = routerLogits(router: router, x: x, numExperts: s.numExperts, hidden: s.hidden)
        let probs = softmax(logits)
        let (idx, w) = selectTopK(logits: logits, probs: probs, k: s.topK,
                                  normTopkProb: s.normTopkProb)
        let eb = offsets(s).expertBytes
        let outs = idx.map { expertForward(shape: s, block: layerImage + $0 * eb, x: x) }
        return (combine(expertOuts: outs, w: w, residual: residual), idx, w)
    }
}
