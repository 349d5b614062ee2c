// nova.relu is outside this path and is refused by name (a standalone
// nova.gelu is planned as a kernel of its own).
module {
  func.func @standalone_gelu(%x: tensor<4x8xf32>) -> tensor<4x8xf32> {
    %g = nova.gelu %x : tensor<4x8xf32>
    return %g : tensor<4x8xf32>
  }
  func.func @relu(%x: tensor<4x8xf32>) -> tensor<4x8xf32> {
    %r = nova.relu %x : tensor<4x8xf32>
    return %r : tensor<4x8xf32>
  }
}
