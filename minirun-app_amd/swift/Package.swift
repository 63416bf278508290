// swift-tools-version:5.9
// HIPBridge: the MLXBridge-shaped Swift surface over the MI355X C-ABI
// (include/minirun_hip.h, libminirun_hip.so).  Build the library first
// (`python minirun-app_amd/build.py`), then
//   swift build -Xlinker -L../lib -Xlinker -rpath -Xlinker <abs path>/minirun-app_amd/lib
// Minirun adds `HIPBridge` as a dependency of ModelAdapters in place of the
// MLX calls these wrappers replace (each wrapper names the one it replaces).
import PackageDescription

let package = Package(
    name: "HIPBridge",
    products: [.library(name: "HIPBridge", targets: ["HIPBridge"])],
    targets: [
        .systemLibrary(name: "CMinirunHIP", path: "Sources/CMinirunHIP"),
        .target(name: "HIPBridge", dependencies: ["CMinirunHIP"], path: "Sources/HIPBridge"),
    ]
)
