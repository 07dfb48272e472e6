// A GDA attention layer over the 4-slot KV cache, driven through the MotifHIP
// entry points: the HIP counterpart of the attention core of the reference's
// grouped forward (swift/Sources/MotifKitMLX/MotifMLXModel.swift:259-524):
// RoPE on q and k, the 4-slot append (update_and_fetch_4), the origin and
// noise dual-V passes and the GDA epilogue, for decode steps and prefill
// chunks.  The q/k/v projections, o_proj and the rest of the block stay with
// the caller, which hands in the projection outputs and gets the epilogue
// output (B, qGroups*gr, S, 2D) back.
//
// As the reference's kernel layer does (MotifMetalKernels.swift:562-593,
// telemetry 193-248), each step tries the fused entry point first, falls back
// to the composed entry points when the fused one reports .unsupported, and
// counts every fallback by reason.  A step that neither covers returns
// .unsupported, so the caller can take its own reference path.
//
// Device memory comes from a caller-supplied MotifHIPDeviceMemory, so this
// file needs no HIP runtime import.  Buffers this layer stops using (a grown
// cache's old slots, a grown workspace) are released only after the copies
// out of them are ordered on the step's stream; an allocator whose release
// is not stream-ordered must synchronise that stream first.

public protocol MotifHIPDeviceMemory: AnyObject {
    /// Device allocation of `bytes`, zero-filled; nil on failure.
    func allocate(bytes: Int) -> UnsafeMutableRawPointer?
    func release(_ pointer: UnsafeMutableRawPointer)
    /// `rows` rows of `rowBytes` bytes from src (row pitch srcPitch) to dst
    /// (row pitch dstPitch), ordered on `stream` (hipMemcpy2DAsync).
    func copyRows(to dst: UnsafeMutableRawPointer, dstPitch: Int, from src: UnsafeRawPointer,
                  srcPitch: Int, rowBytes: Int, rows: Int,
                  stream: UnsafeMutableRawPointer?) -> Bool
}

public enum MotifHIPCacheFormat: Equatable {
    /// fp16/bf16/fp32 rows (B, kGroups, capacity, D) per slot.
    case float(MotifHIPDType)
    /// MLX-affine packed rows: data (B, kGroups, capacity, D*bits/32) uint32,
    /// fp16 scales and biases (B, kGroups, capacity, D/groupSize).
    case quantized(bits: Int, groupSize: Int)
}

/// Head layout of one layer (model.py:563-600): qGroups noise heads, each with
/// gr origin heads, over kGroups KV heads; k_ratio 1.
public struct MotifHIPAttentionShape {
    public var batch: Int
    public var qGroups: Int
    public var gr: Int
    public var kGroups: Int
    public var headDim: Int
    public var activations: MotifHIPDType
    public var theta: Float
    /// RoPE position scale: 1, or MotifHIP.ropePositionScale of the model's
    /// rope_scaling config.
    public var positionScale: Float
    public var originFirst: Bool
    public var scale: Float

    public init(batch: Int, qGroups: Int, gr: Int, kGroups: Int, headDim: Int,
                activations: MotifHIPDType, theta: Float, positionScale: Float = 1,
                originFirst: Bool = false, scale: Float? = nil) {
        self.batch = batch
        self.qGroups = qGroups
        self.gr = gr
        self.kGroups = kGroups
        self.headDim = headDim
        self.activations = activations
        self.theta = theta
        self.positionScale = positionScale
        self.originFirst = originFirst
        self.scale = scale ?? 1.0 / Float(headDim).squareRoot()
    }

    var originHeads: Int { qGroups * gr }
    var elementBytes: Int { activations == .float32 ? 4 : 2 }
}

/// Fallback counts per reason (MotifKernelFallbackTelemetry,
/// MotifMetalKernels.swift:193-248).
public final class MotifHIPFallbackTelemetry {
    public private(set) var counts: [String: Int] = [:]
    public init() {}
    public func record(_ reason: String) { counts[reason, default: 0] += 1 }
}

/// The four slots (k1, k2, v1, v2) of one layer's cache (cache.py:178-545),
/// grown `step` rows at a time with the live rows copied over, as the
/// reference's _grow does (cache.py:245-265).
public final class MotifHIPGroupedCache {
    public static let step = 256
    public let format: MotifHIPCacheFormat
    public let shape: MotifHIPAttentionShape
    public private(set) var offset = 0
    public private(set) var capacity = 0
    private let memory: MotifHIPDeviceMemory
    private var parts: [[UnsafeMutableRawPointer]] = []  // [slot][data, scales, biases]

    public init(format: MotifHIPCacheFormat, shape: MotifHIPAttentionShape,
                memory: MotifHIPDeviceMemory) {
        self.format = format
        self.shape = shape
        self.memory = memory
    }

    deinit {
        for slot in parts { for p in slot { memory.release(p) } }
    }

    /// Bytes of one row of each part of a slot.
    private var partRowBytes: [Int] {
        switch format {
        case .float(let dtype):
            return [shape.headDim * (dtype == .float32 ? 4 : 2)]
        case .quantized(let bits, let groupSize):
            let groups = shape.headDim / groupSize
            return [shape.headDim * bits / 8, groups * 2, groups * 2]
        }
    }

    /// Capacity for `rows` live rows; false if an allocation or copy failed
    /// (the cache is then unchanged).
    public func ensureCapacity(_ rows: Int, stream: UnsafeMutableRawPointer?) -> Bool {
        if rows <= capacity { return true }
        let newCapacity = (rows + Self.step - 1) / Self.step * Self.step
        let planes = shape.batch * shape.kGroups
        var grown: [[UnsafeMutableRawPointer]] = []
        func undo() { for slot in grown { for p in slot { memory.release(p) } } }
        for slot in 0 ..< 4 {
            var slotParts: [UnsafeMutableRawPointer] = []
            for (i, rowBytes) in partRowBytes.enumerated() {
                guard let p = memory.allocate(bytes: planes * newCapacity * rowBytes) else {
                    for q in slotParts { memory.release(q) }
                    undo()
                    return false
                }
                slotParts.append(p)
                if offset > 0 {
                    let ok = memory.copyRows(to: p, dstPitch: newCapacity * rowBytes,
                                             from: parts[slot][i], srcPitch: capacity * rowBytes,
                                             rowBytes: offset * rowBytes, rows: planes,
                                             stream: stream)
                    if !ok {
                        for q in slotParts { memory.release(q) }
                        undo()
                        return false
                    }
                }
            }
            grown.append(slotParts)
        }
        for slot in parts { for p in slot { memory.release(p) } }
        parts = grown
        capacity = newCapacity
        return true
    }

    func advance(by rows: Int) { offset += rows }

    /// Slot i of a float cache.
    func slot(_ i: Int) -> UnsafeMutableRawPointer { parts[i][0] }

    /// Slot i of a packed cache.
    func triple(_ i: Int) -> MotifHIPQuantizedTriple {
        MotifHIPQuantizedTriple(data: parts[i][0].assumingMemoryBound(to: UInt32.self),
                                scales: parts[i][1], biases: parts[i][2])
    }
}

/// One layer's attention over its cache.  sublnWeight (2D values of the
/// activation dtype) and lambdaFull (one fp32 value) are device pointers the
/// caller owns; oneMinusLambdaInit and eps are the layer's constants.
public final class MotifHIPGroupedAttention {
    public let shape: MotifHIPAttentionShape
    public let cache: MotifHIPGroupedCache
    public let telemetry = MotifHIPFallbackTelemetry()
    private let memory: MotifHIPDeviceMemory
    private let sublnWeight: UnsafeRawPointer
    private let lambdaFull: UnsafePointer<Float>
    private let oneMinusLambdaInit: Float
    private let eps: Float
    private var workspace: UnsafeMutableRawPointer?
    private var workspaceBytes = 0
    private var scratch: [Int: (pointer: UnsafeMutableRawPointer, bytes: Int)] = [:]
    private var retired: [UnsafeMutableRawPointer] = []

    public init(shape: MotifHIPAttentionShape, format: MotifHIPCacheFormat,
                memory: MotifHIPDeviceMemory, sublnWeight: UnsafeRawPointer,
                lambdaFull: UnsafePointer<Float>, oneMinusLambdaInit: Float, eps: Float = 1e-6) {
        self.shape = shape
        self.cache = MotifHIPGroupedCache(format: format, shape: shape, memory: memory)
        self.memory = memory
        self.sublnWeight = sublnWeight
        self.lambdaFull = lambdaFull
        self.oneMinusLambdaInit = oneMinusLambdaInit
        self.eps = eps
    }

    deinit {
        if let w = workspace { memory.release(w) }
        for (_, s) in scratch { memory.release(s.pointer) }
        for p in retired { memory.release(p) }
    }

    /// The split workspace grows and is never shrunk; a superseded one is
    /// kept until the layer goes, since a captured graph may still hold it.
    /// New workspaces come zero-filled (their merge counters start at 0).
    private func ensureWorkspace(_ bytes: Int) -> Bool {
        if bytes <= workspaceBytes { return true }
        guard let w = memory.allocate(bytes: bytes) else { return false }
        if let old = workspace { retired.append(old) }
        workspace = w
        workspaceBytes = bytes
        return true
    }

    private func scratchBuffer(_ key: Int, bytes: Int) -> UnsafeMutableRawPointer? {
        if let s = scratch[key], s.bytes >= bytes { return s.pointer }
        guard let p = memory.allocate(bytes: bytes) else { return nil }
        if let old = scratch[key] { retired.append(old.pointer) }
        scratch[key] = (p, bytes)
        return p
    }

    /// One decode step: projections of one token (q (B, 1, qGroups*(gr+1)*D),
    /// k and v (B, 1, 2*kGroups*D)) -> output (B, qGroups*gr, 1, 2D).  The
    /// token's rows land at row `cache.offset`, which then advances by one.
    /// Replaces model.py:590-594, 620-629 and 717-768 for S = 1.
    public func decode(qProj: UnsafeRawPointer, kProj: UnsafeRawPointer,
                       vProj: UnsafeRawPointer, output: UnsafeMutableRawPointer,
                       stream: UnsafeMutableRawPointer?) -> MotifHIPStatus {
        guard shape.qGroups == shape.kGroups else {
            telemetry.record("decode: q_groups != k_groups")
            return .unsupported
        }
        let kvLen = cache.offset + 1
        guard cache.ensureCapacity(kvLen, stream: stream) else { return .hip }
        let ws = MotifHIP.gdaDecodeWorkspaceBytes(batch: shape.batch, kvHeads: shape.kGroups,
                                                  gr: shape.gr, kvLen: kvLen,
                                                  headDim: shape.headDim)
        guard ensureWorkspace(ws) else { return .hip }
        let rowBytes = shape.headDim * shape.elementBytes
        var status: MotifHIPStatus
        switch cache.format {
        case .float(let dtype):
            status = MotifHIP.gdaDecodeFromProjections(
                qProj: qProj, kProj: kProj, vProj: vProj, keys1: cache.slot(0),
                keys2: cache.slot(1), value1: cache.slot(2), value2: cache.slot(3),
                sublnWeight: sublnWeight, lambdaFull: lambdaFull,
                oneMinusLambdaInit: oneMinusLambdaInit, eps: eps, output: output, dtype: dtype,
                batch: shape.batch, kvHeads: shape.kGroups, gr: shape.gr,
                headDim: shape.headDim, kvCapacity: cache.capacity, kvLen: kvLen,
                scale: shape.scale, theta: shape.theta, positionScale: shape.positionScale,
                originFirst: shape.originFirst,
                workspace: workspace, workspaceBytes: workspaceBytes, stream: stream)
            if status == .unsupported {
                telemetry.record("decode: rope_split4 + gda_decode")
                guard let q1 = scratchBuffer(0, bytes: shape.batch * shape.originHeads * rowBytes),
                      let q2 = scratchBuffer(1, bytes: shape.batch * shape.qGroups * rowBytes)
                else { return .hip }
                status = MotifHIP.ropeSplit4(
                    qProj: qProj, kProj: kProj, vProj: vProj, q1: q1, q2: q2,
                    k1: cache.slot(0), k2: cache.slot(1), v1: cache.slot(2), v2: cache.slot(3),
                    dtype: dtype, batch: shape.batch, seqLen: 1, qGroups: shape.qGroups,
                    gr: shape.gr, kGroups: shape.kGroups, kRatio: 1, headDim: shape.headDim,
                    capacity: cache.capacity, row0: cache.offset, pos0: cache.offset,
                    theta: shape.theta, positionScale: shape.positionScale,
                    originFirst: shape.originFirst, stream: stream)
                if status == .ok {
                    status = MotifHIP.gdaDecode(
                        originQueries: q1, noiseQueries: q2, keys1: cache.slot(0),
                        keys2: cache.slot(1), value1: cache.slot(2), value2: cache.slot(3),
                        sublnWeight: sublnWeight, lambdaFull: lambdaFull,
                        oneMinusLambdaInit: oneMinusLambdaInit, eps: eps, output: output,
                        dtype: dtype, batch: shape.batch, kvHeads: shape.kGroups, gr: shape.gr,
                        headDim: shape.headDim, kvCapacity: cache.capacity, kvLen: kvLen,
                        scale: shape.scale, workspace: workspace,
                        workspaceBytes: workspaceBytes, stream: stream)
                }
            }
        case .quantized(let bits, let groupSize):
            status = MotifHIP.gdaDecodeQuantizedFromProjections(
                qProj: qProj, kProj: kProj, vProj: vProj, keys1: cache.triple(0),
                keys2: cache.triple(1), value1: cache.triple(2), value2: cache.triple(3),
                sublnWeight: sublnWeight, lambdaFull: lambdaFull,
                oneMinusLambdaInit: oneMinusLambdaInit, eps: eps, output: output,
                dtype: shape.activations, batch: shape.batch, kvHeads: shape.kGroups,
                gr: shape.gr, headDim: shape.headDim, kvCapacity: cache.capacity,
                kvLen: kvLen, bits: bits, groupSize: groupSize, scale: shape.scale,
                theta: shape.theta, positionScale: shape.positionScale,
                originFirst: shape.originFirst, workspace: workspace,
                workspaceBytes: workspaceBytes, stream: stream)
            if status == .unsupported {
                // The token's roped rows as plain (B, H, 1, D) tensors, then
                // the step that quantises them into row kvLen - 1.
                telemetry.record("decode: rope_split4 + gda_decode_q_append")
                let kvRows = shape.batch * shape.kGroups * rowBytes
                guard let q1 = scratchBuffer(0, bytes: shape.batch * shape.originHeads * rowBytes),
                      let q2 = scratchBuffer(1, bytes: shape.batch * shape.qGroups * rowBytes),
                      let k1 = scratchBuffer(2, bytes: kvRows),
                      let k2 = scratchBuffer(3, bytes: kvRows),
                      let v1 = scratchBuffer(4, bytes: kvRows),
                      let v2 = scratchBuffer(5, bytes: kvRows)
                else { return .hip }
                status = MotifHIP.ropeSplit4(
                    qProj: qProj, kProj: kProj, vProj: vProj, q1: q1, q2: q2, k1: k1, k2: k2,
                    v1: v1, v2: v2, dtype: shape.activations, batch: shape.batch, seqLen: 1,
                    qGroups: shape.qGroups, gr: shape.gr, kGroups: shape.kGroups, kRatio: 1,
                    headDim: shape.headDim, capacity: 1, row0: 0, pos0: cache.offset,
                    theta: shape.theta, positionScale: shape.positionScale,
                    originFirst: shape.originFirst, stream: stream)
                if status == .ok {
                    status = MotifHIP.gdaDecodeQuantizedAppend(
                        originQueries: q1, noiseQueries: q2, newKeys1: k1, newKeys2: k2,
                        newValue1: v1, newValue2: v2, keys1: cache.triple(0),
                        keys2: cache.triple(1), value1: cache.triple(2), value2: cache.triple(3),
                        sublnWeight: sublnWeight, lambdaFull: lambdaFull,
                        oneMinusLambdaInit: oneMinusLambdaInit, eps: eps, output: output,
                        dtype: shape.activations, batch: shape.batch, kvHeads: shape.kGroups,
                        gr: shape.gr, headDim: shape.headDim, kvCapacity: cache.capacity,
                        kvLen: kvLen, bits: bits, groupSize: groupSize, scale: shape.scale,
                        workspace: workspace, workspaceBytes: workspaceBytes, stream: stream)
                }
            }
        }
        if status == .ok { cache.advance(by: 1) }
        return status
    }

    /// One prefill chunk of seqLen tokens over a float cache: projections
    /// (B, seqLen, ...) -> output (B, qGroups*gr, seqLen, 2D), query row s
    /// attending cache rows [0, offset + s].  Replaces model.py:590-594,
    /// 620-629 and the causal fallback 769-807 with gda_post_split.  Packed
    /// caches and shapes without a fused prefill kernel return .unsupported.
    public func prefill(qProj: UnsafeRawPointer, kProj: UnsafeRawPointer,
                        vProj: UnsafeRawPointer, seqLen: Int, output: UnsafeMutableRawPointer,
                        stream: UnsafeMutableRawPointer?) -> MotifHIPStatus {
        guard case .float(let dtype) = cache.format else {
            telemetry.record("prefill: packed cache")
            return .unsupported
        }
        let kvLen = cache.offset + seqLen
        guard cache.ensureCapacity(kvLen, stream: stream) else { return .hip }
        let ws = MotifHIP.gdaPrefillWorkspaceBytes(batch: shape.batch, seqLen: seqLen,
                                                   qGroups: shape.qGroups, gr: shape.gr,
                                                   kGroups: shape.kGroups,
                                                   headDim: shape.headDim, kvLen: kvLen)
        guard ensureWorkspace(ws) else { return .hip }
        let rowBytes = 2 * shape.headDim * shape.elementBytes  // one (s, 2D) output row
        guard let yOrigin = scratchBuffer(10, bytes: shape.batch * shape.originHeads * seqLen * rowBytes),
              let yNoise = scratchBuffer(11, bytes: shape.batch * shape.qGroups * seqLen * rowBytes)
        else { return .hip }
        var status = MotifHIP.gdaPrefillFromProjections(
            qProj: qProj, kProj: kProj, vProj: vProj, keys1: cache.slot(0), keys2: cache.slot(1),
            value1: cache.slot(2), value2: cache.slot(3), outputOrigin: yOrigin,
            outputNoise: yNoise, dtype: dtype, batch: shape.batch, seqLen: seqLen,
            qGroups: shape.qGroups, gr: shape.gr, kGroups: shape.kGroups,
            headDim: shape.headDim, kvCapacity: cache.capacity, offset: cache.offset,
            scale: shape.scale, theta: shape.theta, positionScale: shape.positionScale,
            originFirst: shape.originFirst,
            workspace: workspace, workspaceBytes: workspaceBytes, stream: stream)
        if status == .unsupported {
            telemetry.record("prefill: no fused kernel for this shape")
            return .unsupported
        }
        if status == .ok {
            status = MotifHIP.gdaPostSplit(
                attnO: yOrigin, attnN: yNoise, sublnWeight: sublnWeight, output: output,
                dtype: dtype, batch: shape.batch, qOrigin: shape.originHeads,
                qGroups: shape.qGroups, gr: shape.gr, rows: seqLen,
                channels: 2 * shape.headDim, lambdaFull: lambdaFull,
                oneMinusLambdaInit: oneMinusLambdaInit, eps: eps, stream: stream)
        }
        if status == .ok { cache.advance(by: seqLen) }
        return status
    }
}
