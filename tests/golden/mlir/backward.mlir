// nova.linear_backward (f32) and nova.matmul_backward (bf16 data read through
// widening casts: f32 accumulate, f32 grads).
module {
  func.func @lin_bwd(%go: tensor<40x24xf32>, %x: tensor<40x36xf32>, %w: tensor<36x24xf32>) -> (tensor<40x36xf32>, tensor<36x24xf32>, tensor<24xf32>) {
    %gi, %gw, %gb = nova.linear_backward %go, %x, %w : tensor<40x24xf32>, tensor<40x36xf32>, tensor<36x24xf32>
    return %gi, %gw, %gb : tensor<40x36xf32>, tensor<36x24xf32>, tensor<24xf32>
  }
  func.func @mm_bwd(%g: tensor<64x96xbf16>, %a: tensor<64x128xbf16>, %b: tensor<128x96xbf16>) -> (tensor<64x128xf32>, tensor<128x96xf32>) {
    %gf = nova.cast %g : tensor<64x96xbf16> -> tensor<64x96xf32>
    %af = nova.cast %a : tensor<64x128xbf16> -> tensor<64x128xf32>
    %bf = nova.cast %b : tensor<128x96xbf16> -> tensor<128x96xf32>
    %ga, %gb = nova.matmul_backward %gf, %af, %bf : tensor<64x96xf32>, tensor<64x128xf32>, tensor<128x96xf32>
    return %ga, %gb : tensor<64x128xf32>, tensor<128x96xf32>
  }
}
