// Config-2 form at a small size: linalg.batch_matmul with bf16 ins and f32
// outs over a zero fill, and the same product written as nova.matmul on
// widened operands.
module {
  func.func @bmm(%A: tensor<4x128x96xbf16>, %B: tensor<4x96x160xbf16>) -> tensor<4x128x160xf32> {
    %cst = arith.constant 0.000000e+00 : f32
    %e = tensor.empty() : tensor<4x128x160xf32>
    %C = linalg.fill ins(%cst : f32) outs(%e : tensor<4x128x160xf32>) -> tensor<4x128x160xf32>
    %r = linalg.batch_matmul ins(%A, %B : tensor<4x128x96xbf16>, tensor<4x96x160xbf16>)
                             outs(%C : tensor<4x128x160xf32>) -> tensor<4x128x160xf32>
    return %r : tensor<4x128x160xf32>
  }
  func.func @bmm_nova(%A: tensor<4x128x96xbf16>, %B: tensor<4x96x160xbf16>) -> tensor<4x128x160xf32> {
    %a = nova.cast %A : tensor<4x128x96xbf16> -> tensor<4x128x96xf32>
    %b = nova.cast %B : tensor<4x96x160xbf16> -> tensor<4x96x160xf32>
    %r = nova.matmul %a, %b : tensor<4x128x96xf32>, tensor<4x96x160xf32>
    return %r : tensor<4x128x160xf32>
  }
}
