// hipcheck — HIPMoE (libm1moe_hip on the GPU) against the Swift oracle
// (Sources/M1MoEOracle) on one seeded synthetic MoE layer of a model's
// shape: the north star's parity bar, top-K indices bit-exact and the layer
// output within 1e-2 relative L2 (f32 accumulation on both sides).
//
//   swift run hipcheck configs/olmoe-1b-7b.json [seed]
//
// The layer is drawn like the benchmark's configs: nibbles uniform in 0..15,
// group scales |N(0, 0.02)|, biases N(0, 0.01), router N(0, 0.02), all bf16;
// x and the residual N(0, 1).  Not compiled in this source tree (no Swift
// toolchain); the repository's own GPU tests run the same checks through
// Python over the C ABI (tests/test_gpu_decode.py).

import CM1MoEHIP
import Foundation
import M1MoE
import M1MoEOracle

/// splitmix64: a seeded stream of 64-bit values.
struct SplitMix64 {
    var state: UInt64
    mutating func next() -> UInt64 {
        state &+= 0x9E37_79B9_7F4A_7C15
        var z = state
        z = (z ^ (z >> 30)) &* 0xBF58_476D_1CE4_E5B9
        z = (z ^ (z >> 27)) &* 0x94D0_49BB_1331_11EB
        return z ^ (z >> 31)
    }
    /// uniform in (0, 1)
    mutating func uniform() -> Double { (Double(next() >> 11) + 0.5) / 9_007_199_254_740_992.0 }
    /// N(0, 1) by Box-Muller
    mutating func normal() -> Double {
        let u1 = uniform(), u2 = uniform()
        return (-2 * log(u1)).squareRoot() * cos(2 * Double.pi * u2)
    }
}

/// f32 -> bf16, round to nearest even (finite inputs).
func bf16(_ f: Float) -> UInt16 {
    let u = f.bitPattern
    return UInt16(truncatingIfNeeded: (u &+ 0x7FFF &+ ((u >> 16) & 1)) >> 16)
}

func relL2(_ a: [Float], _ b: [Float]) -> Double {
    var num = 0.0, den = 0.0
    for i in 0 ..< a.count {
        let d = Double(a[i]) - Double(b[i])
        num += d * d
        den += Double(b[i]) * Double(b[i])
    }
    return (num / max(den, 1e-300)).squareRoot()
}

func check(_ rc: Int32, _ what: String) {
    if rc != 0 {
        print("\(what) failed: status \(rc): \(String(cString: m1moe_last_error()))")
        exit(1)
    }
}

let args = CommandLine.arguments
guard args.count >= 2 else {
    print("usage: hipcheck CONFIG.json [seed]")
    exit(2)
}
let spec = try ModelSpec.load(from: URL(fileURLWithPath: args[1]))
var rng = SplitMix64(state: args.count >= 3 ? UInt64(args[2]) ?? 2026 : 2026)
let shape = MoEOracleShape(hidden: spec.hiddenDim, numExperts: spec.moe.numExperts,
                           topK: spec.moe.topK, intermediate: spec.moe.intermediateDim,
                           groupSize: spec.quantization.groupSize,
                           normTopkProb: spec.moe.normTopkProb)
let off = MoEOracle.offsets(shape)
let h = shape.hidden, E = shape.numExperts, K = shape.topK

// one layer image: E expert blocks in the layout of ModelSpec.swift:36-52
var image = [UInt8](repeating: 0, count: off.expertBytes * E)
image.withUnsafeMutableBytes { raw in
    for e in 0 ..< E {
        let blk = raw.baseAddress! + e * off.expertBytes
        let parts: [(Int, Int, Int)] = [(off.gateW, off.gateS, off.gateB),
                                        (off.upW, off.upS, off.upB),
                                        (off.downW, off.downS, off.downB)]
        for (wOff, sOff, bOff) in parts {
            let words = (sOff - wOff) / 4, groups = (bOff - sOff) / 2
            let w = (blk + wOff).assumingMemoryBound(to: UInt32.self)
            for i in 0 ..< words { w[i] = UInt32(truncatingIfNeeded: rng.next()) }
            let s = (blk + sOff).assumingMemoryBound(to: UInt16.self)
            let b = (blk + bOff).assumingMemoryBound(to: UInt16.self)
            for g in 0 ..< groups {
                s[g] = bf16(Float(abs(rng.normal()) * 0.02))
                b[g] = bf16(Float(rng.normal() * 0.01))
            }
        }
    }
}
let router = (0 ..< E * h).map { _ in bf16(Float(rng.normal() * 0.02)) }
let x = (0 ..< h).map { _ in Float(rng.normal()) }
let residual = (0 ..< h).map { _ in Float(rng.normal()) }

// the GPU: layer 0 of a context of the model's shape
let moe = try HIPMoE(spec: spec)
try moe.uploadLayer(0, image: Data(image))
router.withUnsafeBufferPointer {
    check(m1moe_upload_router(moe.ctx, 0, $0.baseAddress, UInt64(E * h)), "m1moe_upload_router")
}
var got = [Float](repeating: 0, count: h)
try x.withUnsafeBufferPointer { xp in
    try residual.withUnsafeBufferPointer { rp in
        try got.withUnsafeMutableBufferPointer { op in
            try moe.forward(layer: 0, x: xp.baseAddress!, residual: rp.baseAddress!,
                            out: op.baseAddress!)
        }
    }
}
// the GPU's routing (the optional top-K outputs of m1moe_moe_decode)
var dX: UnsafeMutableRawPointer?, dOut: UnsafeMutableRawPointer?
var dIdx: UnsafeMutableRawPointer?, dW: UnsafeMutableRawPointer?
check(m1moe_alloc(moe.ctx, UInt64(4 * h), &dX), "m1moe_alloc")
check(m1moe_alloc(moe.ctx, UInt64(4 * h), &dOut), "m1moe_alloc")
check(m1moe_alloc(moe.ctx, UInt64(4 * K), &dIdx), "m1moe_alloc")
check(m1moe_alloc(moe.ctx, UInt64(4 * K), &dW), "m1moe_alloc")
x.withUnsafeBytes { check(m1moe_copy_h2d(moe.ctx, dX, $0.baseAddress, UInt64($0.count)), "copy") }
check(m1moe_moe_decode(moe.ctx, 0, dX, Int32(M1MOE_F32), nil,
                       dOut!.assumingMemoryBound(to: Float.self),
                       dIdx!.assumingMemoryBound(to: Int32.self),
                       dW!.assumingMemoryBound(to: Float.self)), "m1moe_moe_decode")
var gIdx = [Int32](repeating: 0, count: K), gW = [Float](repeating: 0, count: K)
gIdx.withUnsafeMutableBytes { check(m1moe_copy_d2h(moe.ctx, $0.baseAddress, dIdx, UInt64($0.count)), "copy") }
gW.withUnsafeMutableBytes { check(m1moe_copy_d2h(moe.ctx, $0.baseAddress, dW, UInt64($0.count)), "copy") }
check(m1moe_sync(moe.ctx), "m1moe_sync")
for p in [dX, dOut, dIdx, dW] { _ = m1moe_free(moe.ctx, p) }

// the oracle
let want = image.withUnsafeBytes { img in
    router.withUnsafeBufferPointer { r in
        MoEOracle.decode(shape: shape, layerImage: img.baseAddress!, router: r.baseAddress!,
                         x: x, residual: residual)
    }
}
let rel = relL2(got, want.out)
let idxOK = gIdx.map { Int($0) } == want.idx
var wErr: Float = 0
for j in 0 ..< K { wErr = max(wErr, abs(gW[j] - want.w[j]) / max(abs(want.w[j]), 1e-30)) }
print("\(spec.name): top-\(K) \(idxOK ? "equal" : "DIFFERENT") (GPU \(gIdx), oracle \(want.idx)), "
      + "weights rel err \(wErr), output rel L2 \(rel)")
exit(idxOK && wErr <= 2e-6 && rel <= 1e-2 ? 0 : 1)
