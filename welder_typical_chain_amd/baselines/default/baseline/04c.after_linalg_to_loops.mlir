// Loop structure of the unfused path's kernels on gfx950 (variant tile128x128_wave64x32),
// with this problem's bounds: batch 1, M 8192, N 128, K 64.  Each func is one HIP kernel; scf.parallel is its grid.
module attributes {wtc.target = "gfx950", wtc.path = "unfused"} {
  // chain_tile_kernel<f16,f32,logits,128x128>: grid 64 x 512 threads, 137984 bytes of LDS
  func.func @kernel0() {
    %c0 = arith.constant 0 : index
    %c1 = arith.constant 1 : index
    %grid = arith.constant 64 : index
    %c2 = arith.constant 2 : index
    scf.parallel (%wg) = (%c0) to (%grid) step (%c1) {
      %nk = arith.constant 1 : index
      %ks = arith.constant 4 : index
      %tm = arith.constant 128 : index
      %tn = arith.constant 128 : index
      // workgroup -> (row block, column tile) of 128x128, XCD-aware order
      scf.for %kt = %c0 to %nk step %c1 {  // k-tiles of 64 elements: direct-to-LDS buffer loads of k-tile kt+3 into the LDS ring
        scf.for %s = %c0 to %ks step %c1 {  // LDS fragment reads (B: ds_read_b64_tr), v_mfma_f32_32x32x16_f16, f32 accumulators
        }
      }
      scf.for %r = %c0 to %tm step %c1 {  // logits scale*acc in f32: 16-byte stores
        scf.for %n = %c0 to %tn step %c1 {
        }
      }
      scf.reduce
    }
    return
  }
  // rowmax_kernel: grid 8192 x 256 threads, 16 bytes of LDS
  func.func @kernel1() {
    %c0 = arith.constant 0 : index
    %c1 = arith.constant 1 : index
    %grid = arith.constant 8192 : index
    %c2 = arith.constant 2 : index
    scf.parallel (%wg) = (%c0) to (%grid) step (%c1) {
      %n = arith.constant 128 : index
      scf.for %j = %c0 to %n step %c1 {  // row max over row wg of 8192 rows
      }
      scf.reduce
    }
    return
  }
  // expsub_kernel: grid 8192 x 256 threads, 0 bytes of LDS
  func.func @kernel2() {
    %c0 = arith.constant 0 : index
    %c1 = arith.constant 1 : index
    %grid = arith.constant 8192 : index
    %c2 = arith.constant 2 : index
    scf.parallel (%wg) = (%c0) to (%grid) step (%c1) {
      %n = arith.constant 128 : index
      scf.for %j = %c0 to %n step %c1 {  // exp(x - max) over row wg of 8192 rows
      }
      scf.reduce
    }
    return
  }
  // rowsum_kernel: grid 8192 x 256 threads, 16 bytes of LDS
  func.func @kernel3() {
    %c0 = arith.constant 0 : index
    %c1 = arith.constant 1 : index
    %grid = arith.constant 8192 : index
    %c2 = arith.constant 2 : index
    scf.parallel (%wg) = (%c0) to (%grid) step (%c1) {
      %n = arith.constant 128 : index
      scf.for %j = %c0 to %n step %c1 {  // row sum over row wg of 8192 rows
      }
      scf.reduce
    }
    return
  }
  // rowdiv_kernel<f32>: grid 8192 x 256 threads, 0 bytes of LDS
  func.func @kernel4() {
    %c0 = arith.constant 0 : index
    %c1 = arith.constant 1 : index
    %grid = arith.constant 8192 : index
    %c2 = arith.constant 2 : index
    scf.parallel (%wg) = (%c0) to (%grid) step (%c1) {
      %n = arith.constant 128 : index
      scf.for %j = %c0 to %n step %c1 {  // divide over row wg of 8192 rows
      }
      scf.reduce
    }
    return
  }
}
