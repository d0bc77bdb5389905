// RUN: not %tb-opt %s --tb-verify-scope 2>&1 | FileCheck %s

// A #tb.shared encoding that breaks the reference's SharedEncodingAttr
// verifier (lib/IR/TBAttrs.cpp:120-148): negative max_phase, and no cga
// owner. The module is refused as it is read, before any pass runs.
#bad_shared = #tb.shared<order = [1, 0], perPhase = 0, maxPhase = -3, transposed = false, swizzlingByteWidth = 7>

module attributes {"tb.num-warps" = 4 : i64, "tb.requested-stages" = 2 : i64} {
  func.func @kernel(%A: memref<64x32xf16>, %B: memref<32x64xf16>,
                    %C: memref<64x64xf32>) {
    tb.matmul %A, %B, %C {block_m = 64 : i64, block_n = 64 : i64,
                          block_k = 32 : i64, exact_tile = true}
      : memref<64x32xf16>, memref<32x64xf16>, memref<64x64xf32>
    func.return
  }
}

// CHECK: error: invalid `#tb.shared`: expected parameter `cga`, found the end
