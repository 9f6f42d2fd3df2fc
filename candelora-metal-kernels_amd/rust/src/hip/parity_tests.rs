// cpu_vs_hip_parity_* tests: the `rocm` build's counterpart of the crate's
// cpu_vs_metal_parity_* tests (src/iq2_matmul.rs:1065-1313), on the same
// inputs (the parity case: m = 2, out_dim = 7, in_dim = 320, seeded codes,
// every d = 1).  Included inside the crate's test module, whose helpers it
// uses (lcg_fill, deterministic_x, force_f16_one_per_block,
// iq2_matmul_reference, rowwise_quant_dequant_w8a8,
// iq2_matmul_reference_w8a8), with the module's cfg widened to
// `all(test, any(feature = "metal", feature = "rocm"))` (and the cfg of the
// per-block size constants behind `bytes_per_block` / `scales_per_block` to
// `any(feature = "metal", feature = "rocm")`, as the `rocm` body needs too):
//
//     #[cfg(feature = "rocm")]
//     mod hip_parity {
//         include!("hip/parity_tests.rs");
//     }
//
// The GPU path sums in another order than the CPU loop, and with d = 1 the
// outputs reach a few thousand, where the CPU loop's own fp32 result is up to
// 2.2e-3 from the exact product (IQ3_S).  So every case holds the GPU result
// to the crate's bar (2e-3; W8A8 3e-3) of the exact product, and to that bar
// plus the CPU loop's own distance from the exact product of the CPU result.
// Where the margins measured on MI355X leave room (every format but IQ3_S in
// mode Off: at most 1.34e-3; W8A8 at most 0.98e-3), the crate's own form,
// |gpu - cpu| <= bar, is asserted as well.  Not built in this repository (no
// Rust toolchain in its image); tests/test_gpu_variants.py and
// tests/test_gpu_parity.py hold the same checks through the C ABI.

use super::*;
use crate::activation_quant::{ActivationQuantConfig, ActivationQuantMode};
use candle_core::{Device, Result, Tensor};

const M: usize = 2;
const N: usize = 7;
const K: usize = 320;

/// The crate's parity-case inputs for `variant`.
fn parity_inputs(variant: Iq2MatmulVariant) -> (Vec<f32>, Vec<u8>, Vec<u8>) {
    let blocks = N * K.div_ceil(IQ2_QK);
    let mut codes = lcg_fill(blocks * variant.bytes_per_block(), 0xA11CE5ED);
    let mut scales = lcg_fill(blocks * variant.scales_per_block(), 0xC0FFEE12);
    force_f16_one_per_block(&mut scales, variant.scales_per_block());
    if let Some(b) = codes.last_mut() {
        *b = 0x5A;
    }
    (deterministic_x(M, K), codes, scales)
}

/// The HIP result: CPU tensors, which the `rocm` body stages to the GPU.
fn hip_result(
    x: &[f32],
    codes: &[u8],
    scales: &[u8],
    variant: Iq2MatmulVariant,
    mode: ActivationQuantMode,
) -> Result<Vec<f32>> {
    let dev = Device::Cpu;
    let x = Tensor::from_slice(x, (M, K), &dev)?;
    let codes = Tensor::from_slice(codes, codes.len(), &dev)?;
    let scales = Tensor::from_slice(scales, scales.len(), &dev)?;
    let quant = ActivationQuantConfig { mode, strict: false };
    iq2_matmul_with_activation_quant(&x, &codes, &scales, N, K, variant, &quant)?
        .reshape((M * N,))?
        .to_vec1::<f32>()
}

/// The exact weights, column by column: the CPU reference on one-hot rows
/// returns each column exactly (every weight d (2s+1) g / 8, or d (1+2s) g, is
/// an fp32 value, and a one-hot row sums a single product with zeros).
fn exact_weights(codes: &[u8], scales: &[u8], variant: Iq2MatmulVariant) -> Vec<f64> {
    let mut w = vec![0f64; N * K];
    let mut e = vec![0f32; K];
    for k in 0..K {
        e.fill(0.0);
        e[k] = 1.0;
        let col = iq2_matmul_reference(&e, 1, N, K, codes, scales, variant);
        for n in 0..N {
            w[n * K + k] = col[n] as f64;
        }
    }
    w
}

fn exact_product(x: &[f32], w: &[f64]) -> Vec<f64> {
    let mut y = vec![0f64; M * N];
    for r in 0..M {
        for n in 0..N {
            y[r * N + n] = (0..K).map(|k| x[r * K + k] as f64 * w[n * K + k]).sum();
        }
    }
    y
}

fn max_diff(a: &[f32], b: &[f64]) -> f64 {
    a.iter().zip(b).map(|(&u, &v)| (u as f64 - v).abs()).fold(0.0, f64::max)
}

fn check(variant: Iq2MatmulVariant, mode: ActivationQuantMode, bar: f64, direct: bool) -> Result<()> {
    let (x, codes, scales) = parity_inputs(variant);
    let (cpu, x_used) = match mode {
        ActivationQuantMode::W8A8 => (
            iq2_matmul_reference_w8a8(&x, M, N, K, &codes, &scales, variant),
            rowwise_quant_dequant_w8a8(&x, M, K),
        ),
        _ => (iq2_matmul_reference(&x, M, N, K, &codes, &scales, variant), x.clone()),
    };
    let exact = exact_product(&x_used, &exact_weights(&codes, &scales, variant));
    let gpu = hip_result(&x, &codes, &scales, variant, mode)?;
    let cpu_own = max_diff(&cpu, &exact);
    let gpu_exact = max_diff(&gpu, &exact);
    let gpu_cpu = max_diff(&gpu, &cpu.iter().map(|&v| v as f64).collect::<Vec<_>>());
    assert!(gpu_exact <= bar, "{variant:?} {mode:?}: |hip - exact| = {gpu_exact} > {bar}");
    assert!(
        gpu_cpu <= bar + cpu_own,
        "{variant:?} {mode:?}: |hip - cpu| = {gpu_cpu} > {bar} + {cpu_own} (the CPU loop's own error)"
    );
    if direct {
        assert!(gpu_cpu <= bar, "{variant:?} {mode:?}: |hip - cpu| = {gpu_cpu} > {bar}");
    }
    Ok(())
}

#[test]
fn cpu_vs_hip_parity_iq2_xxs() -> Result<()> {
    check(Iq2MatmulVariant::Iq2Xxs, ActivationQuantMode::Off, 2e-3, true)
}

#[test]
fn cpu_vs_hip_parity_iq2_xs() -> Result<()> {
    check(Iq2MatmulVariant::Iq2Xs, ActivationQuantMode::Off, 2e-3, true)
}

#[test]
fn cpu_vs_hip_parity_iq2_s() -> Result<()> {
    check(Iq2MatmulVariant::Iq2S, ActivationQuantMode::Off, 2e-3, true)
}

#[test]
fn cpu_vs_hip_parity_iq3_s() -> Result<()> {
    // |hip - cpu| read 2.44e-3 on MI355X: the CPU loop is itself 2.17e-3 from
    // the exact product on this case, so only the exact-product form holds
    check(Iq2MatmulVariant::Iq3S, ActivationQuantMode::Off, 2e-3, false)
}

#[test]
fn cpu_vs_hip_parity_w8a8_iq2_xxs() -> Result<()> {
    check(Iq2MatmulVariant::Iq2Xxs, ActivationQuantMode::W8A8, 3e-3, true)
}

#[test]
fn cpu_vs_hip_parity_w8a8_iq2_xs() -> Result<()> {
    check(Iq2MatmulVariant::Iq2Xs, ActivationQuantMode::W8A8, 3e-3, true)
}

#[test]
fn cpu_vs_hip_parity_w8a8_iq2_s() -> Result<()> {
    check(Iq2MatmulVariant::Iq2S, ActivationQuantMode::W8A8, 3e-3, true)
}

#[test]
fn cpu_vs_hip_parity_w8a8_iq3_s() -> Result<()> {
    check(Iq2MatmulVariant::Iq3S, ActivationQuantMode::W8A8, 3e-3, true)
}
