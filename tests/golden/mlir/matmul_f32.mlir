// Config-1 form: f32 matmul (exact f32 kernel) and a bias-folded nova.linear.
module {
  func.func @mm(%A: tensor<256x256xf32>, %B: tensor<256x256xf32>) -> tensor<256x256xf32> {
    %r = nova.matmul %A, %B : tensor<256x256xf32>, tensor<256x256xf32>
    return %r : tensor<256x256xf32>
  }
  func.func @lin(%x: tensor<33x70xf32>, %w: tensor<70x45xf32>, %b: tensor<45xf32>) -> tensor<33x45xf32> {
    %y = nova.linear %x, %w, %b : tensor<33x70xf32>, tensor<70x45xf32>, tensor<45xf32>
    return %y : tensor<33x45xf32>
  }
}
