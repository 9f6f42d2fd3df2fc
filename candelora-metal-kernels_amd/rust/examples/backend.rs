// Backend selection for examples/iq2_matmul_bench.rs (`--backend metal|hip`),
// to be added as examples/backend.rs and included with `mod backend;`.  The
// bench parses the flag with `Backend::from_arg`, creates its device with
// `Backend::device`, and keeps its timed loop unchanged.  With `hip` the device
// is the CPU: the `rocm` bodies of src/iq2_matmul.rs stage the tensors into
// device buffers per call, so these latencies include PCIe copies; bench.py in
// the HIP build reports device-resident throughput.  Not built here.
use candle_core::{Device, Result};

#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum Backend {
    Metal,
    Hip,
}

impl Backend {
    pub fn from_arg(s: &str) -> Result<Self> {
        match s {
            "metal" => Ok(Backend::Metal),
            "hip" => Ok(Backend::Hip),
            other => candle_core::bail!("unknown --backend {other}: expected metal or hip"),
        }
    }

    pub fn device(self) -> Result<Device> {
        match self {
            Backend::Metal => Device::new_metal(0),
            Backend::Hip => {
                if cfg!(feature = "rocm") {
                    Ok(Device::Cpu)
                } else {
                    candle_core::bail!("--backend hip needs a build with --features rocm")
                }
            }
        }
    }

    /// The cargo feature that builds this backend.
    pub fn feature(self) -> &'static str {
        match self {
            Backend::Metal => "metal",
            Backend::Hip => "rocm",
        }
    }
}
