// swift-tools-version:5.9
// The C module over libmoehip.so (the MI355X MoE layer). FFAI's package
// depends on it by path and links the library from ffai_amd/:
//
//   dependencies: [.package(path: "<repo>/swift")],
//   .target(name: "FFAI", dependencies: [.product(name: "CMoEHIP", package: "CMoEHIP")],
//           linkerSettings: [.unsafeFlags(["-L<repo>/ffai_amd", "-Xlinker", "-rpath",
//                                          "-Xlinker", "<repo>/ffai_amd"])])
//
// (FFAI's own targets are declared in its Package.swift:40-95.)
import PackageDescription

let package = Package(
    name: "CMoEHIP",
    products: [.library(name: "CMoEHIP", targets: ["CMoEHIP"])],
    targets: [.systemLibrary(name: "CMoEHIP", path: "CMoEHIP")]
)
