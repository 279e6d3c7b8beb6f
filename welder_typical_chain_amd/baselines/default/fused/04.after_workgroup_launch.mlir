// Launches of the fused Matmul -> row-Softmax chain on gfx950, exchange path: one launch region per HIP kernel
// with its grid, block and LDS (static + dynamic bytes, the workgroup attribution).  The bodies are the
// kernels of the code object 05.out.gfx950.hsaco (library /root/repo/welder_typical_chain_amd/libwtc_hip.so), variant tile128x128_wave64x32.
module attributes {gpu.container_module, wtc.target = "gfx950", wtc.path = "exchange", wtc.compute_units = 256 : i32} {
  func.func @chain(%a: memref<8192x64xf16>, %b: memref<64x128xf16>, %out: memref<8192x128xf32>, %ws: memref<69888xi8>) {
    %c1 = arith.constant 1 : index
    %g0 = arith.constant 64 : index
    %t0 = arith.constant 512 : index
    gpu.launch blocks(%bx0, %by0, %bz0) in (%gx0 = %g0, %gy0 = %c1, %gz0 = %c1) threads(%tx0, %ty0, %tz0) in (%sx0 = %t0, %sy0 = %c1, %sz0 = %c1) workgroup(%lds0 : memref<137984xi8, 3>) {
      // body: chain_tile_kernel<f16,f32,exchange,128x128>
      gpu.terminator
    }
    return
  }
}
